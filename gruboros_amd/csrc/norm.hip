// Fused residual add + RMSNorm, forward and backward, for gfx950.
//
// Reference: mingru/minLM.py:119-125 (x = mingru(norm(x)) + x), :130
// (x = ff(ff_norm(x)) + x), :137 (final norm); the norms are
// torch.nn.RMSNorm(dim) (:67, :69, :74) with eps = None, i.e. the fp32
// machine epsilon 2^-23 (the caller passes it; it is not the activation
// dtype's epsilon). Per row of D elements:
//   xn = x + delta                  (the residual stream, fp32)
//   r  = 1 / sqrt(mean(xn^2) + eps)
//   y  = xn * r * w                 (bf16 or fp32, the next op's input)
//   y_lo = bf16(y - bf16(y))        (optional, with a bf16 y: y as a hi/lo
//                                    pair, hi + lo = y to ~2^-16 relative,
//                                    for products that need fp32 accuracy)
// Backward, with dy the gradient of y and dres that of xn from later
// residual uses:
//   g  = dy * w,  m = mean(g * xn * r)
//   dxn = r * (g - xn * r * m) + dres     (= dx = ddelta)
//   dw  = sum over rows of dy * xn * r
//
// One wave per row: lane l holds columns {4 l + 256 i} (16-byte fp32
// vectors), so every row access is a contiguous 1 KiB per wave step and the
// row reduction is a wave reduction. Workgroups are grid-strided over rows;
// w stays in registers, and the backward accumulates dw per lane, reduces it
// over the workgroup in LDS and writes one partial row per workgroup; a
// second kernel sums the partials.

#include <algorithm>

#include "mg_common.h"

namespace mg {
namespace norm {

constexpr int kWaves = 8;                 // rows in flight per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kColsPerStep = 256;         // 64 lanes x 4 columns

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T>
__device__ __forceinline__ f4 load_cols(const T* p, int col, int D) {
  return col < D ? io4<T>::load(p + col) : io4<T>::fill(0.0f);
}

// The fp32 residual stream is touched once per pass and read back only much
// later (the next block's norm, the backward), so the forward's x loads and
// x_out stores and the backward's loads of the saved x carry the
// non-temporal hint; the bf16 outputs (read by the next product) do not.
// Measured in the cfg3 step: 11.50 -> 11.39 ms.
typedef float f32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4 load_cols_stream(const float* p, int col, int D) {
  if (col >= D) return io4<float>::fill(0.0f);
  const f32x4_nt x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(p + col));
  f4 r;
  r.v[0] = x[0]; r.v[1] = x[1]; r.v[2] = x[2]; r.v[3] = x[3];
  return r;
}
__device__ __forceinline__ void store4_stream(float* p, const f4& r) {
  const f32x4_nt x = {r.v[0], r.v[1], r.v[2], r.v[3]};
  __builtin_nontemporal_store(x, reinterpret_cast<f32x4_nt*>(p));
}

template <typename Td, typename Ty, int kSteps>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_fwd_kernel(
    const float* __restrict__ x, const Td* __restrict__ delta, const float* __restrict__ w,
    float* __restrict__ x_out, Ty* __restrict__ y, bf16_t* __restrict__ y_lo, int64_t ldy,
    float* __restrict__ rstd, int64_t N, int D, float eps) {
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  f4 wv[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) wv[i] = load_cols(w, 4 * lane + kColsPerStep * i, D);
  const float inv_d = 1.0f / static_cast<float>(D);
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave; row < N;
       row += static_cast<int64_t>(gridDim.x) * kWaves) {
    const int64_t base = row * D;
    f4 xv[kSteps];
#pragma unroll
    for (int i = 0; i < kSteps; ++i) xv[i] = load_cols_stream(x + base, 4 * lane + kColsPerStep * i, D);
    if (delta) {
#pragma unroll
      for (int i = 0; i < kSteps; ++i) {
        const f4 dv = load_cols(delta + base, 4 * lane + kColsPerStep * i, D);
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[i].v[j] += dv.v[j];
      }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kSteps; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += xv[i].v[j] * xv[i].v[j];
    ss = wave_sum(ss);
    const float r = __builtin_amdgcn_rsqf(ss * inv_d + eps);
    const int64_t ybase = row * ldy;
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int col = 4 * lane + kColsPerStep * i;
      if (col < D) {
        f4 yv;
#pragma unroll
        for (int j = 0; j < 4; ++j) yv.v[j] = xv[i].v[j] * r * wv[i].v[j];
        io4<Ty>::store(y + ybase + col, yv);
        if (y_lo) {
          f4 lo;  // y - bf16(y) is exact in fp32
#pragma unroll
          for (int j = 0; j < 4; ++j) lo.v[j] = yv.v[j] - bf16_to_f32(f32_to_bf16(yv.v[j]));
          io4<bf16_t>::store(y_lo + ybase + col, lo);
        }
        if (delta && x_out) store4_stream(x_out + base + col, xv[i]);
      }
    }
    if (lane == 0 && rstd) rstd[row] = r;
  }
}

template <typename Tg, typename Td, int kSteps>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_bwd_kernel(
    const float* __restrict__ xn, const float* __restrict__ w, const float* __restrict__ rstd,
    const Tg* __restrict__ dy, const float* __restrict__ dy_scale, const float* __restrict__ dres,
    float* __restrict__ dx, Td* __restrict__ ddelta, float* __restrict__ dw_part, int64_t N, int D) {
  __shared__ f4 s_dw[kWaves][64];
  // dy times a device scalar (the upstream gradient of a loss): the same fp32
  // product a separate pass over dy would store; x 1 is exact
  const float sc = dy_scale ? *dy_scale : 1.0f;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  f4 wv[kSteps], dwa[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    wv[i] = load_cols(w, 4 * lane + kColsPerStep * i, D);
    dwa[i] = io4<float>::fill(0.0f);
  }
  const float inv_d = 1.0f / static_cast<float>(D);
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave; row < N;
       row += static_cast<int64_t>(gridDim.x) * kWaves) {
    const int64_t base = row * D;
    const float r = rstd[row];
    f4 xh[kSteps], gv[kSteps], dyv[kSteps];
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int col = 4 * lane + kColsPerStep * i;
      xh[i] = load_cols_stream(xn + base, col, D);
      dyv[i] = load_cols(dy + base, col, D);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dyv[i].v[j] *= sc;
        xh[i].v[j] *= r;
        gv[i].v[j] = dyv[i].v[j] * wv[i].v[j];
        dot += gv[i].v[j] * xh[i].v[j];
      }
    }
    const float m = wave_sum(dot) * inv_d;
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int col = 4 * lane + kColsPerStep * i;
      if (col < D) {
        f4 d = dres ? io4<float>::load(dres + base + col) : io4<float>::fill(0.0f);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          d.v[j] += r * (gv[i].v[j] - xh[i].v[j] * m);
          dwa[i].v[j] += dyv[i].v[j] * xh[i].v[j];
        }
        if (dx) io4<float>::store(dx + base + col, d);
        // a bf16 ddelta rounds stochastically (mg_common.h)
        if (ddelta) io4<Td>::store_grad(ddelta + base + col, d, static_cast<uint32_t>(base + col), 0x7c39u);
      }
    }
  }
  // dw: sum the waves' partials in LDS (one 256-column step at a time), one
  // partial row per workgroup.
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    s_dw[wave][lane] = dwa[i];
    __syncthreads();
    if (wave == 0) {
      f4 acc = s_dw[0][lane];
#pragma unroll
      for (int q = 1; q < kWaves; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc.v[j] += s_dw[q][lane].v[j];
      const int col = 4 * lane + kColsPerStep * i;
      if (col < D) io4<float>::store(dw_part + static_cast<int64_t>(blockIdx.x) * D + col, acc);
    }
    __syncthreads();
  }
}

// Register steps per lane: ceil(D / 256) rounded up to a power of two (the
// extra columns are masked).
inline int steps_for(int D) {
  const int need = (D + kColsPerStep - 1) / kColsPerStep;
  int s = 1;
  while (s < need) s <<= 1;
  return s;
}

// Workgroups for a row count: two per CU of a 256-CU device at most, so the
// backward's partial-dw rows stay few.
inline int grid_for(int64_t N) {
  const int64_t want = (N + kWaves - 1) / kWaves;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(want, 512)));
}

template <typename Td, typename Ty>
int launch_fwd(const float* x, const void* delta, const float* w, float* x_out, void* y, void* y_lo, int64_t ldy,
               float* rstd, int64_t N, int D, float eps, hipStream_t st) {
  const int grid = grid_for(N);
  const Td* dl = static_cast<const Td*>(delta);
  Ty* yy = static_cast<Ty*>(y);
  switch (steps_for(D)) {
#define MG_NORM_FWD(S)                                                                                  \
  case S:                                                                                              \
    hipLaunchKernelGGL((add_rmsnorm_fwd_kernel<Td, Ty, S>), dim3(grid), dim3(kThreads), 0, st, x, dl, w, \
                       x_out, yy, static_cast<bf16_t*>(y_lo), ldy, rstd, N, D, eps);                   \
    break;
    MG_NORM_FWD(1) MG_NORM_FWD(2) MG_NORM_FWD(4) MG_NORM_FWD(8) MG_NORM_FWD(16)
#undef MG_NORM_FWD
    default:
      return fail(MG_ERR_ARG, "mg_add_rmsnorm_fwd: D=%d unsupported (D <= 4096)", D);
  }
  return check_launch("mg_add_rmsnorm_fwd");
}

template <typename Tg, typename Td>
int launch_bwd(const float* xn, const float* w, const float* rstd, const void* dy, const float* dy_scale,
               const float* dres, float* dx, void* ddelta, float* dw, float* dw_part, int64_t N, int D,
               hipStream_t st) {
  const int grid = grid_for(N);
  const Tg* g = static_cast<const Tg*>(dy);
  Td* dd = static_cast<Td*>(ddelta);
  switch (steps_for(D)) {
#define MG_NORM_BWD(S)                                                                                   \
  case S:                                                                                               \
    hipLaunchKernelGGL((add_rmsnorm_bwd_kernel<Tg, Td, S>), dim3(grid), dim3(kThreads), 0, st, xn, w, rstd, \
                       g, dy_scale, dres, dx, dd, dw_part, N, D);                                       \
    break;
    MG_NORM_BWD(1) MG_NORM_BWD(2) MG_NORM_BWD(4) MG_NORM_BWD(8) MG_NORM_BWD(16)
#undef MG_NORM_BWD
    default:
      return fail(MG_ERR_ARG, "mg_add_rmsnorm_bwd: D=%d unsupported (D <= 4096)", D);
  }
  launch_reduce_partials(dw_part, grid, D, dw, st);
  return check_launch("mg_add_rmsnorm_bwd");
}

inline int check_dtype(const char* fn, const char* name, int dt) {
  if (dt != MG_F32 && dt != MG_BF16) return fail(MG_ERR_DTYPE, "%s: %s dtype %d unsupported", fn, name, dt);
  return MG_OK;
}

inline int check_ptr(const char* fn, const char* name, const void* p, size_t align, bool required) {
  if (!p) return required ? fail(MG_ERR_ARG, "%s: %s is NULL", fn, name) : MG_OK;
  if (!aligned(p, align)) return fail(MG_ERR_ARG, "%s: %s not %zu-byte aligned", fn, name, align);
  return MG_OK;
}

}  // namespace norm
}  // namespace mg

using namespace mg;

extern "C" size_t mg_add_rmsnorm_bwd_workspace_bytes(int64_t N, int D) {
  return static_cast<size_t>(norm::grid_for(N)) * static_cast<size_t>(std::max(D, 0)) * sizeof(float);
}

extern "C" int mg_add_rmsnorm_fwd(const float* x, int delta_dtype, const void* delta, const float* w,
                                  float* x_out, int y_dtype, void* y, void* y_lo, int64_t ldy, float* rstd,
                                  int64_t N, int D, float eps, void* stream) {
  const char* fn = "mg_add_rmsnorm_fwd";
  int rc;
  if (N < 1 || D < 4 || D % 4) return fail(MG_ERR_ARG, "%s: bad shape N=%lld D=%d (D %% 4 == 0)", fn, (long long)N, D);
  if ((rc = norm::check_ptr(fn, "x", x, 16, true))) return rc;
  if ((rc = norm::check_ptr(fn, "w", w, 16, true))) return rc;
  if ((rc = norm::check_ptr(fn, "y", y, y_dtype == MG_F32 ? 16 : 8, true))) return rc;
  if ((rc = norm::check_ptr(fn, "rstd", rstd, 4, false))) return rc;
  if ((rc = norm::check_dtype(fn, "y", y_dtype))) return rc;
  if (ldy < D || ldy % 4) return fail(MG_ERR_ARG, "%s: ldy=%lld must be >= D=%d and a multiple of 4", fn, (long long)ldy, D);
  if (y_lo) {
    if (y_dtype != MG_BF16) return fail(MG_ERR_DTYPE, "%s: y_lo needs a bf16 y", fn);
    if ((rc = norm::check_ptr(fn, "y_lo", y_lo, 8, true))) return rc;
  }
  if (delta) {
    if ((rc = norm::check_dtype(fn, "delta", delta_dtype))) return rc;
    if ((rc = norm::check_ptr(fn, "delta", delta, delta_dtype == MG_F32 ? 16 : 8, true))) return rc;
    if ((rc = norm::check_ptr(fn, "x_out", x_out, 16, true))) return rc;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool dbf = delta && delta_dtype == MG_BF16;
  if (y_dtype == MG_BF16)
    return dbf ? norm::launch_fwd<bf16_t, bf16_t>(x, delta, w, x_out, y, y_lo, ldy, rstd, N, D, eps, st)
               : norm::launch_fwd<float, bf16_t>(x, delta, w, x_out, y, y_lo, ldy, rstd, N, D, eps, st);
  return dbf ? norm::launch_fwd<bf16_t, float>(x, delta, w, x_out, y, nullptr, ldy, rstd, N, D, eps, st)
             : norm::launch_fwd<float, float>(x, delta, w, x_out, y, nullptr, ldy, rstd, N, D, eps, st);
}

extern "C" int mg_add_rmsnorm_bwd_scaled(const float* xn, const float* w, const float* rstd, int dy_dtype,
                                         const void* dy, const float* dy_scale, const float* dres, float* dx,
                                         int ddelta_dtype, void* ddelta, float* dw, int64_t N, int D,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "mg_add_rmsnorm_bwd";
  int rc;
  if (N < 1 || D < 4 || D % 4) return fail(MG_ERR_ARG, "%s: bad shape N=%lld D=%d (D %% 4 == 0)", fn, (long long)N, D);
  if ((rc = norm::check_ptr(fn, "xn", xn, 16, true))) return rc;
  if ((rc = norm::check_ptr(fn, "w", w, 16, true))) return rc;
  if ((rc = norm::check_ptr(fn, "rstd", rstd, 4, true))) return rc;
  if ((rc = norm::check_dtype(fn, "dy", dy_dtype))) return rc;
  if ((rc = norm::check_ptr(fn, "dy", dy, dy_dtype == MG_F32 ? 16 : 8, true))) return rc;
  if ((rc = norm::check_ptr(fn, "dy_scale", dy_scale, 4, false))) return rc;
  if ((rc = norm::check_ptr(fn, "dres", dres, 16, false))) return rc;
  if ((rc = norm::check_ptr(fn, "dx", dx, 16, false))) return rc;
  if ((rc = norm::check_ptr(fn, "dw", dw, 16, true))) return rc;
  if (ddelta) {
    if ((rc = norm::check_dtype(fn, "ddelta", ddelta_dtype))) return rc;
    if ((rc = norm::check_ptr(fn, "ddelta", ddelta, ddelta_dtype == MG_F32 ? 16 : 8, true))) return rc;
  }
  const size_t need = mg_add_rmsnorm_bwd_workspace_bytes(N, D);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 16))
    return fail(MG_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu (or misaligned)", fn, workspace_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const bool gbf = dy_dtype == MG_BF16, dbf = ddelta && ddelta_dtype == MG_BF16;
  if (gbf)
    return dbf ? norm::launch_bwd<bf16_t, bf16_t>(xn, w, rstd, dy, dy_scale, dres, dx, ddelta, dw, part, N, D, st)
               : norm::launch_bwd<bf16_t, float>(xn, w, rstd, dy, dy_scale, dres, dx, ddelta, dw, part, N, D, st);
  return dbf ? norm::launch_bwd<float, bf16_t>(xn, w, rstd, dy, dy_scale, dres, dx, ddelta, dw, part, N, D, st)
             : norm::launch_bwd<float, float>(xn, w, rstd, dy, dy_scale, dres, dx, ddelta, dw, part, N, D, st);
}

extern "C" int mg_add_rmsnorm_bwd(const float* xn, const float* w, const float* rstd, int dy_dtype, const void* dy,
                                  const float* dres, float* dx, int ddelta_dtype, void* ddelta, float* dw,
                                  int64_t N, int D, void* workspace, size_t workspace_bytes, void* stream) {
  return mg_add_rmsnorm_bwd_scaled(xn, w, rstd, dy_dtype, dy, nullptr, dres, dx, ddelta_dtype, ddelta, dw, N, D,
                                   workspace, workspace_bytes, stream);
}
