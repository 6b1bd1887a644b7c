// Column sums over the token rows: the bias gradients of the FeedForward
// linears (reference mingru/minLM.py:17-23, autograd of nn.Linear's bias),
// one of them fused with GELU's backward, and the reduction of per-workgroup
// partial rows that the RMSNorm weight gradient also uses.
//
//   mg_column_sum:   out[c] = sum_n x[n, c]                        (x bf16 / fp32)
//   mg_gelu_bwd:     dpre[n, c] = bf16(dh[n, c] gelu'(pre[n, c]))  (dh fp32 or
//                                 bf16; dpre rounded stochastically, mg_common.h)
//                    dbias[c]   = sum_n dpre[n, c]   (of the rounded values,
//                                 as summing the bf16 tensor gives)
// Both make one pass over the rows: workgroup (cb, rg) owns 2048 columns
// (8 per thread, one 16-byte bf16 vector) of the rows rg, rg + RG, ...,
// and writes one partial row; launch_reduce_partials sums the RG partial
// rows in a fixed order (the results do not depend on scheduling).

#include <algorithm>

#include "mg_common.h"

namespace mg {
namespace colsum {

constexpr int kThreads = 256;
constexpr int kVecC = 8;                          // columns per thread
constexpr int kCols = kThreads * kVecC;           // columns per workgroup

// Row groups (= partial rows): about `wgs` workgroups in all. The column sum
// runs best at 512 (two per CU); the GELU backward, with its erf and exp per
// element, at 1024 (measured: 5% faster at 4096 columns, 11% at 8192).
constexpr int kSumWgs = 512, kGeluWgs = 1024;
inline int row_groups(int64_t N, int C, int wgs = kSumWgs) {
  const int64_t col_blocks = std::max<int64_t>(1, (C + kCols - 1) / kCols);
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(N, std::max<int64_t>(1, wgs / col_blocks))));
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]);
template <>
__device__ __forceinline__ void load8<bf16_t>(const bf16_t* p, float (&v)[8]) {
  const uint4 x = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = __uint_as_float(w[q] << 16);
    v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Non-temporal 16-byte load of 8 bf16 values. The GELU backward's inputs (the
// saved pre-activation and the gradient dh just written, 134 MB each at cfg3)
// are read once; loaded with the hint the cfg3 step measured 11.31 -> 11.19 ms.
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void load8_stream(const bf16_t* p, float (&v)[8]) {
  const u32x4_nt x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = __uint_as_float(x[q] << 16);
    v[2 * q + 1] = __uint_as_float(x[q] & 0xffff0000u);
  }
}

// The column sums of workgroup (bx, by) of a bx x gy grid.
template <typename T>
__device__ __forceinline__ void colsum_block(const T* __restrict__ x, int64_t ld, int64_t N, int C,
                                             float* __restrict__ part, int bx, int by, int gy) {
  const int c = bx * kCols + threadIdx.x * kVecC;
  if (c >= C) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll 4
  for (int64_t n = by; n < N; n += gy) {
    float v[8];
    load8<T>(x + n * ld + c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e];
  }
  float* o = part + static_cast<int64_t>(by) * C + c;
  reinterpret_cast<float4*>(o)[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  reinterpret_cast<float4*>(o)[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void colsum_kernel(const T* __restrict__ x, int64_t ld, int64_t N, int C,
                                                          float* __restrict__ part) {
  colsum_block<T>(x, ld, N, C, part, blockIdx.x, blockIdx.y, gridDim.y);
}

// The GELU backward of workgroup (bx, by) of a bx x gy grid.
template <typename Tg>
__device__ __forceinline__ void gelu_bwd_block(const Tg* __restrict__ dh, int64_t ld_dh,
                                               const bf16_t* __restrict__ pre, int64_t ld_pre,
                                               bf16_t* __restrict__ dpre, int64_t ld_out, int64_t N, int C,
                                               float* __restrict__ part, int bx, int by, int gy) {
  const int c = bx * kCols + threadIdx.x * kVecC;
  if (c >= C) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t n = by; n < N; n += gy) {  // not unrolled: measured fastest
    float g[8], x[8];
    if constexpr (sizeof(Tg) == 2)
      load8_stream(reinterpret_cast<const bf16_t*>(dh + n * ld_dh + c), g);
    else
      load8<Tg>(dh + n * ld_dh + c, g);
    load8_stream(pre + n * ld_pre + c, x);
    uint32_t w[4];
    const uint32_t idx = static_cast<uint32_t>(n * C + c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      w[q] = pack_bf16x2_sr(g[2 * q] * gelu_grad(x[2 * q]), g[2 * q + 1] * gelu_grad(x[2 * q + 1]), idx + 2 * q,
                            0xaf6cu);
      acc[2 * q] += __uint_as_float(w[q] << 16);
      acc[2 * q + 1] += __uint_as_float(w[q] & 0xffff0000u);
    }
    *reinterpret_cast<uint4*>(dpre + n * ld_out + c) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (part) {
    float* o = part + static_cast<int64_t>(by) * C + c;
    reinterpret_cast<float4*>(o)[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    reinterpret_cast<float4*>(o)[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

template <typename Tg>
__global__ __launch_bounds__(kThreads) void gelu_bwd_kernel(const Tg* __restrict__ dh, int64_t ld_dh,
                                                            const bf16_t* __restrict__ pre, int64_t ld_pre,
                                                            bf16_t* __restrict__ dpre, int64_t ld_out, int64_t N,
                                                            int C, float* __restrict__ part) {
  gelu_bwd_block<Tg>(dh, ld_dh, pre, ld_pre, dpre, ld_out, N, C, part, blockIdx.x, blockIdx.y, gridDim.y);
}

// The FeedForward backward's elementwise work in one launch: the GELU
// backward with the first bias gradient's partials (workgroups [0, g1): a
// cb1 x rg1 grid) and the second bias gradient's column-sum partials of dy
// (workgroups [g1, g1 + cb2 rg2)).
template <typename Tg>
__global__ __launch_bounds__(kThreads) void ff_bias_bwd_kernel(const Tg* __restrict__ dh, int64_t ld_dh,
                                                               const bf16_t* __restrict__ pre, int64_t ld_pre,
                                                               bf16_t* __restrict__ dpre, int64_t ld_out, int C1,
                                                               float* __restrict__ part1, int cb1, int rg1,
                                                               const bf16_t* __restrict__ dy, int64_t ld_dy, int C2,
                                                               float* __restrict__ part2, int cb2, int rg2,
                                                               int64_t N) {
  const int bid = blockIdx.x, g1 = cb1 * rg1;
  if (bid < g1)
    gelu_bwd_block<Tg>(dh, ld_dh, pre, ld_pre, dpre, ld_out, N, C1, part1, bid % cb1, bid / cb1, rg1);
  else
    colsum_block<bf16_t>(dy, ld_dy, N, C2, part2, (bid - g1) % cb2, (bid - g1) / cb2, rg2);
}

// out[c] = sum_p part[p][c]: 16 columns (4 lanes x 4) by 64 row lanes per
// workgroup; each row lane sums every 64th partial row, then a fixed-order
// tree over the row lanes in LDS.
__device__ __forceinline__ void reduce_partials_block(const float* __restrict__ part, int P, int C,
                                                      float* __restrict__ out, int bx) {
  __shared__ float4 s[64][4];
  const int cl = threadIdx.x % 4, rl = threadIdx.x / 4;
  const int c = bx * 16 + cl * 4;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (c < C) {
#pragma unroll 4
    for (int p = rl; p < P; p += 64) {
      const float4 v = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(p) * C + c);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
  }
  s[rl][cl] = acc;
  __syncthreads();
#pragma unroll
  for (int h = 32; h > 0; h >>= 1) {
    if (rl < h) {
      const float4 o = s[rl + h][cl];
      float4& m = s[rl][cl];
      m.x += o.x; m.y += o.y; m.z += o.z; m.w += o.w;
    }
    __syncthreads();
  }
  if (rl == 0 && c < C) *reinterpret_cast<float4*>(out + c) = s[0][cl];
}

__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ part, int P, int C,
                                                              float* __restrict__ out) {
  reduce_partials_block(part, P, C, out, blockIdx.x);
}

// Two reductions in one launch: workgroups [0, (C1 + 15) / 16) reduce set 1.
__global__ __launch_bounds__(256) void reduce_partials2_kernel(const float* __restrict__ part1, int P1, int C1,
                                                               float* __restrict__ out1,
                                                               const float* __restrict__ part2, int P2, int C2,
                                                               float* __restrict__ out2) {
  const int n1 = (C1 + 15) / 16;
  if (static_cast<int>(blockIdx.x) < n1) reduce_partials_block(part1, P1, C1, out1, blockIdx.x);
  else reduce_partials_block(part2, P2, C2, out2, blockIdx.x - n1);
}

}  // namespace colsum

int launch_reduce_partials(const float* part, int P, int C, float* out, hipStream_t st) {
  hipLaunchKernelGGL(colsum::reduce_partials_kernel, dim3((C + 15) / 16), dim3(256), 0, st, part, P, C, out);
  return MG_OK;
}

}  // namespace mg

using namespace mg;

extern "C" size_t mg_column_sum_workspace_bytes(int64_t N, int C) {
  if (N < 1 || C < 1) return 16;
  // sized for the GELU backward's row groups, which covers the column sum's
  return static_cast<size_t>(std::max(colsum::row_groups(N, C), colsum::row_groups(N, C, colsum::kGeluWgs))) *
         static_cast<size_t>(std::max(C, 0)) * sizeof(float);
}

extern "C" int mg_column_sum(int dtype, const void* x, int64_t ld, int64_t N, int C, float* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
  const char* fn = "mg_column_sum";
  if (!x || !out) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (N < 1 || C < 8 || C % 8 || ld < C || ld % 8) return fail(MG_ERR_ARG, "%s: bad shape N=%lld C=%d ld=%lld", fn,
                                                               (long long)N, C, (long long)ld);
  if (dtype != MG_F32 && dtype != MG_BF16) return fail(MG_ERR_DTYPE, "%s: dtype %d unsupported", fn, dtype);
  if (!aligned(x, 16) || !aligned(out, 16)) return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  const int RG = colsum::row_groups(N, C);
  if (!workspace || workspace_bytes < mg_column_sum_workspace_bytes(N, C) || !aligned(workspace, 16))
    return fail(MG_ERR_WORKSPACE, "%s: workspace too small or misaligned", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const dim3 grid((C + colsum::kCols - 1) / colsum::kCols, RG);
  if (dtype == MG_BF16)
    hipLaunchKernelGGL(colsum::colsum_kernel<bf16_t>, grid, dim3(colsum::kThreads), 0, st,
                       static_cast<const bf16_t*>(x), ld, N, C, part);
  else
    hipLaunchKernelGGL(colsum::colsum_kernel<float>, grid, dim3(colsum::kThreads), 0, st,
                       static_cast<const float*>(x), ld, N, C, part);
  launch_reduce_partials(part, RG, C, out, st);
  return check_launch(fn);
}

extern "C" int mg_gelu_bwd(int dh_dtype, const void* dh, int64_t ld_dh, const void* pre, int64_t ld_pre, void* dpre,
                           int64_t ld_out, float* dbias, int64_t N, int C, void* workspace, size_t workspace_bytes,
                           void* stream) {
  const char* fn = "mg_gelu_bwd";
  if (!dh || !pre || !dpre) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (dh_dtype != MG_F32 && dh_dtype != MG_BF16) return fail(MG_ERR_DTYPE, "%s: dh dtype %d unsupported", fn, dh_dtype);
  if (N < 1 || C < 8 || C % 8 || ld_dh < C || ld_pre < C || ld_out < C || ld_dh % 8 || ld_pre % 8 || ld_out % 8)
    return fail(MG_ERR_ARG, "%s: bad shape N=%lld C=%d", fn, (long long)N, C);
  if (!aligned(dh, 16) || !aligned(pre, 16) || !aligned(dpre, 16) || (dbias && !aligned(dbias, 16)))
    return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  const int RG = colsum::row_groups(N, C, colsum::kGeluWgs);
  if (dbias && (!workspace || workspace_bytes < mg_column_sum_workspace_bytes(N, C) || !aligned(workspace, 16)))
    return fail(MG_ERR_WORKSPACE, "%s: workspace too small or misaligned", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = dbias ? static_cast<float*>(workspace) : nullptr;
  const dim3 grid((C + colsum::kCols - 1) / colsum::kCols, RG);
  if (dh_dtype == MG_BF16)
    hipLaunchKernelGGL(colsum::gelu_bwd_kernel<bf16_t>, grid, dim3(colsum::kThreads), 0, st,
                       static_cast<const bf16_t*>(dh), ld_dh, static_cast<const bf16_t*>(pre), ld_pre,
                       static_cast<bf16_t*>(dpre), ld_out, N, C, part);
  else
    hipLaunchKernelGGL(colsum::gelu_bwd_kernel<float>, grid, dim3(colsum::kThreads), 0, st,
                       static_cast<const float*>(dh), ld_dh, static_cast<const bf16_t*>(pre), ld_pre,
                       static_cast<bf16_t*>(dpre), ld_out, N, C, part);
  if (dbias) launch_reduce_partials(part, RG, C, dbias, st);
  return check_launch(fn);
}

extern "C" size_t mg_ff_bias_bwd_workspace_bytes(int64_t N, int C1, int C2) {
  if (N < 1 || C1 < 1 || C2 < 1) return 16;
  return (static_cast<size_t>(colsum::row_groups(N, C1, colsum::kGeluWgs)) * C1 +
          static_cast<size_t>(colsum::row_groups(N, C2)) * C2) * sizeof(float);
}

extern "C" int mg_ff_bias_bwd(int dh_dtype, const void* dh, int64_t ld_dh, const void* pre, int64_t ld_pre,
                              void* dpre, int64_t ld_out, float* db1, int64_t N, int C1, const void* dy,
                              int64_t ld_dy, float* db2, int C2, void* workspace, size_t workspace_bytes,
                              void* stream) {
  const char* fn = "mg_ff_bias_bwd";
  if (!dh || !pre || !dpre || !db1 || !dy || !db2) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (dh_dtype != MG_F32 && dh_dtype != MG_BF16) return fail(MG_ERR_DTYPE, "%s: dh dtype %d unsupported", fn, dh_dtype);
  if (N < 1 || C1 < 8 || C1 % 8 || ld_dh < C1 || ld_pre < C1 || ld_out < C1 || ld_dh % 8 || ld_pre % 8 ||
      ld_out % 8 || C2 < 8 || C2 % 8 || ld_dy < C2 || ld_dy % 8)
    return fail(MG_ERR_ARG, "%s: bad shape N=%lld C1=%d C2=%d", fn, (long long)N, C1, C2);
  if (!aligned(dh, 16) || !aligned(pre, 16) || !aligned(dpre, 16) || !aligned(db1, 16) || !aligned(dy, 16) ||
      !aligned(db2, 16))
    return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  if (!workspace || workspace_bytes < mg_ff_bias_bwd_workspace_bytes(N, C1, C2) || !aligned(workspace, 16))
    return fail(MG_ERR_WORKSPACE, "%s: workspace too small or misaligned", fn);
  const int rg1 = colsum::row_groups(N, C1, colsum::kGeluWgs), rg2 = colsum::row_groups(N, C2);
  const int cb1 = (C1 + colsum::kCols - 1) / colsum::kCols, cb2 = (C2 + colsum::kCols - 1) / colsum::kCols;
  float* part1 = static_cast<float*>(workspace);
  float* part2 = part1 + static_cast<size_t>(rg1) * C1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(cb1 * rg1 + cb2 * rg2);
  if (dh_dtype == MG_BF16)
    hipLaunchKernelGGL(colsum::ff_bias_bwd_kernel<bf16_t>, grid, dim3(colsum::kThreads), 0, st,
                       static_cast<const bf16_t*>(dh), ld_dh, static_cast<const bf16_t*>(pre), ld_pre,
                       static_cast<bf16_t*>(dpre), ld_out, C1, part1, cb1, rg1, static_cast<const bf16_t*>(dy),
                       ld_dy, C2, part2, cb2, rg2, N);
  else
    hipLaunchKernelGGL(colsum::ff_bias_bwd_kernel<float>, grid, dim3(colsum::kThreads), 0, st,
                       static_cast<const float*>(dh), ld_dh, static_cast<const bf16_t*>(pre), ld_pre,
                       static_cast<bf16_t*>(dpre), ld_out, C1, part1, cb1, rg1, static_cast<const bf16_t*>(dy),
                       ld_dy, C2, part2, cb2, rg2, N);
  hipLaunchKernelGGL(colsum::reduce_partials2_kernel, dim3((C1 + 15) / 16 + (C2 + 15) / 16), dim3(256), 0, st,
                     part1, rg1, C1, db1, part2, rg2, C2, db2);
  return check_launch(fn);
}
