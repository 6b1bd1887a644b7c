// fp32 -> bf16 hi/lo pairs, the operand form of mg_gemm's MG_GEMM_HILO
// products: out[r, c] = hi = bf16(x[r, c]), out[r, cols + c] =
// bf16(x[r, c] - hi). hi + lo equals x to ~2^-16 relative (x - hi is exact in
// fp32). Used for the weights of the accurate products (once per weight
// update) and for the fp32 scan output entering to_out (reference
// mingru/minGRU.py:71).

#include "mg_common.h"

namespace mg {
namespace convert {

__global__ __launch_bounds__(256) void split_hilo_kernel(const float* __restrict__ x, int64_t ldx, int64_t rows,
                                                         int cols, bf16_t* __restrict__ out, int64_t ldo) {
  const int q = cols / 4;  // 4-column groups per row
  const int64_t n = rows * q;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / q;
    const int c = static_cast<int>(i - r * q) * 4;
    const f4 v = io4<float>::load(x + r * ldx + c);
    f4 lo;
#pragma unroll
    for (int j = 0; j < 4; ++j) lo.v[j] = v.v[j] - bf16_to_f32(f32_to_bf16(v.v[j]));
    io4<bf16_t>::store(out + r * ldo + c, v);
    io4<bf16_t>::store(out + r * ldo + cols + c, lo);
  }
}

// fp32 -> three bf16 limbs h = bf16(x), m = bf16(x - h), l = bf16(x - h - m)
// (each difference is exact in fp32, so h + m + l == x wherever l stays a
// normal bf16 value), written as nseg segments, segment s holding limb
// (pattern >> 2s) & 3 (0 h, 1 m, 2 l). stack_rows 0: segments side by side
// along the columns, out[r, s cols + c] (K-contiguous operands); 1: stacked
// along the rows, out[s rows + r, c] (MN-contiguous operands). Two operands
// split with the patterns (h, m, h, m, l, h) and (h, h, m, m, h, l) make one
// plain bf16 product over 6K the sum of the six limb products down to
// 2^-16 relative (hh, mh, hm, mm, lh, hl): fp32 accuracy on MFMA.
// V values per thread (8 where cols % 8 == 0 and out is 16-byte aligned: one
// 16-byte store per segment; else 4); IDX: the index type (32-bit where the
// thread count allows).
template <int V, typename IDX>
__global__ __launch_bounds__(256) void split_limbs_kernel(const float* __restrict__ x, int64_t ldx, IDX rows,
                                                          int cols, int pattern, int nseg, int stack_rows,
                                                          bf16_t* __restrict__ out, int64_t ldo) {
  const IDX q = cols / V;
  const IDX n = rows * q;
  for (IDX i = blockIdx.x * static_cast<IDX>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<IDX>(gridDim.x) * blockDim.x) {
    const IDX r = i / q;
    const int c = static_cast<int>(i - r * q) * V;
    const fv<V> v = iov<float, V>::load(x + static_cast<int64_t>(r) * ldx + c);
    fv<V> limb[3];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float h = bf16_to_f32(f32_to_bf16(v.v[j]));
      const float r1 = v.v[j] - h;
      const float m = bf16_to_f32(f32_to_bf16(r1));
      limb[0].v[j] = h;
      limb[1].v[j] = m;
      limb[2].v[j] = r1 - m;  // rounded to bf16 by the store
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s >= nseg) break;
      const int which = (pattern >> (2 * s)) & 3;
      const fv<V> w = which == 0 ? limb[0] : which == 1 ? limb[1] : limb[2];
      bf16_t* o = stack_rows ? out + (static_cast<int64_t>(s) * rows + r) * ldo + c
                             : out + static_cast<int64_t>(r) * ldo + static_cast<int64_t>(s) * cols + c;
      iov<bf16_t, V>::store(o, w);
    }
  }
}

// fp32 -> bf16 with stochastic rounding (gradients entering a bf16 product).
__global__ __launch_bounds__(256) void round_sr_kernel(const float* __restrict__ x, int64_t n4, bf16_t* __restrict__ out,
                                                       uint32_t salt) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n4;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    io4<bf16_t>::store_grad(out + 4 * i, io4<float>::load(x + 4 * i), static_cast<uint32_t>(4 * i), salt);
}

}  // namespace convert
}  // namespace mg

using namespace mg;

extern "C" int mg_split_hilo(const float* x, int64_t ldx, int64_t rows, int cols, void* out, int64_t ldo,
                             void* stream) {
  const char* fn = "mg_split_hilo";
  if (!x || !out) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (rows < 0 || cols < 0 || cols % 4) return fail(MG_ERR_ARG, "%s: bad shape rows=%lld cols=%d (cols %% 4 == 0)", fn,
                                                   (long long)rows, cols);
  if (ldx < cols || ldx % 4 || ldo < 2 * static_cast<int64_t>(cols) || ldo % 4)
    return fail(MG_ERR_ARG, "%s: bad strides ldx=%lld ldo=%lld", fn, (long long)ldx, (long long)ldo);
  if (!aligned(x, 16) || !aligned(out, 8)) return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  if (rows == 0 || cols == 0) return MG_OK;
  const int64_t n = rows * (cols / 4);
  const int blocks = static_cast<int>(std::min<int64_t>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(convert::split_hilo_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x, ldx,
                     rows, cols, static_cast<bf16_t*>(out), ldo);
  return check_launch(fn);
}

extern "C" int mg_split_limbs(const float* x, int64_t ldx, int64_t rows, int cols, int pattern, int nseg,
                              int stack_rows, void* out, int64_t ldo, void* stream) {
  const char* fn = "mg_split_limbs";
  if (!x || !out) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (rows < 0 || cols < 0 || cols % 4) return fail(MG_ERR_ARG, "%s: bad shape rows=%lld cols=%d (cols %% 4 == 0)", fn,
                                                   (long long)rows, cols);
  if (nseg < 1 || nseg > 8) return fail(MG_ERR_ARG, "%s: nseg %d outside [1, 8]", fn, nseg);
  for (int s = 0; s < nseg; ++s)
    if (((pattern >> (2 * s)) & 3) == 3) return fail(MG_ERR_ARG, "%s: pattern names limb 3 at segment %d", fn, s);
  if (ldx < cols || ldx % 4 || ldo % 4 || ldo < (stack_rows ? cols : static_cast<int64_t>(nseg) * cols))
    return fail(MG_ERR_ARG, "%s: bad strides ldx=%lld ldo=%lld", fn, (long long)ldx, (long long)ldo);
  if (!aligned(x, 16) || !aligned(out, 8)) return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  if (rows == 0 || cols == 0) return MG_OK;
  const bool wide = cols % 8 == 0 && ldo % 8 == 0 && aligned(out, 16);
  const int64_t n = rows * (cols / (wide ? 8 : 4));
  const int blocks = static_cast<int>(std::min<int64_t>((n + 255) / 256, 8192));
  const int sr = stack_rows ? 1 : 0;
  bf16_t* o = static_cast<bf16_t*>(out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n + 256LL * blocks < (int64_t(1) << 31)) {  // every thread index fits in 32 bits
    const int r32 = static_cast<int>(rows);
    if (wide) hipLaunchKernelGGL((convert::split_limbs_kernel<8, int>), dim3(blocks), dim3(256), 0, st, x, ldx, r32, cols, pattern, nseg, sr, o, ldo);
    else hipLaunchKernelGGL((convert::split_limbs_kernel<4, int>), dim3(blocks), dim3(256), 0, st, x, ldx, r32, cols, pattern, nseg, sr, o, ldo);
  } else {
    if (wide) hipLaunchKernelGGL((convert::split_limbs_kernel<8, int64_t>), dim3(blocks), dim3(256), 0, st, x, ldx, rows, cols, pattern, nseg, sr, o, ldo);
    else hipLaunchKernelGGL((convert::split_limbs_kernel<4, int64_t>), dim3(blocks), dim3(256), 0, st, x, ldx, rows, cols, pattern, nseg, sr, o, ldo);
  }
  return check_launch(fn);
}

extern "C" int mg_round_bf16_sr(const float* x, int64_t n, void* out, uint32_t salt, void* stream) {
  const char* fn = "mg_round_bf16_sr";
  if (!x || !out) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (n < 0 || n % 4) return fail(MG_ERR_ARG, "%s: n=%lld must be a non-negative multiple of 4", fn, (long long)n);
  if (!aligned(x, 16) || !aligned(out, 8)) return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  if (n == 0) return MG_OK;
  const int64_t n4 = n / 4;
  const int blocks = static_cast<int>(std::min<int64_t>((n4 + 255) / 256, 4096));
  hipLaunchKernelGGL(convert::round_sr_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x, n4,
                     static_cast<bf16_t*>(out), salt);
  return check_launch(fn);
}
