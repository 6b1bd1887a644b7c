// Fused log-softmax + cross-entropy (mean over rows) with its gradient.
//
// Reference: mingru/minLM.py:146-149, F.cross_entropy(logits.transpose(1, 2),
// labels) with the default mean reduction over the B*T positions
// (labels = ids[:, 1:], :94-95). Per row n of V logits:
//   lse_n  = max_j l_nj + log(sum_j exp(l_nj - max))
//   loss_n = lse_n - l_n,label
//   dl_nj  = (exp(l_nj - lse_n) - [j == label]) * scale     (scale = 1/N)
// The gradient is produced in the same pass (the loss is linear in its
// upstream gradient, which the caller applies afterwards), so the logits are
// read once and never re-read by a backward softmax.
//
// One wave per row: lane l holds classes {4 l + 256 i}; row reductions are
// wave reductions. Each workgroup writes the sum of its rows' losses to
// loss_part[blockIdx] (summed by the caller in a fixed order).

#include <algorithm>
#include <math.h>

#include "mg_common.h"

namespace mg {
namespace ce {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename Tl, typename Td, int kSteps>
__global__ __launch_bounds__(kThreads) void ce_kernel(const Tl* __restrict__ logits, const int64_t* __restrict__ labels,
                                                      Td* __restrict__ dlogits, float* __restrict__ loss_part,
                                                      int* __restrict__ bad_label, int64_t N, int V, float scale) {
  __shared__ float s_loss[kWaves];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  float acc = 0.0f;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave; row < N;
       row += static_cast<int64_t>(gridDim.x) * kWaves) {
    const Tl* lp = logits + row * V;
    const int64_t lab = labels[row];
    f4 x[kSteps];
    float m = -INFINITY, picked = 0.0f;
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int col = 4 * lane + 256 * i;
      x[i] = col < V ? io4<Tl>::load(lp + col) : io4<float>::fill(-INFINITY);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m = fmaxf(m, x[i].v[j]);
        if (col + j == lab) picked = x[i].v[j];
      }
    }
    m = wave_max(m);
    picked = wave_sum(picked);  // l_label (one lane holds it)
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kSteps; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[i].v[j] = expf(x[i].v[j] - m);  // softmax numerator
        s += x[i].v[j];
      }
    s = wave_sum(s);
    if (lane == 0) {
      acc += logf(s) + m - picked;  // lse - l_label
      if ((lab < 0 || lab >= V) && bad_label) atomicOr(bad_label, 1);
    }
    const float inv_s = 1.0f / s;
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int col = 4 * lane + 256 * i;
      if (col < V) {
        f4 d;
#pragma unroll
        for (int j = 0; j < 4; ++j) d.v[j] = (x[i].v[j] * inv_s - (col + j == lab ? 1.0f : 0.0f)) * scale;
        io4<Td>::store_grad(dlogits + row * V + col, d, static_cast<uint32_t>(row * V + col), 0x8d4au);
      }
    }
  }
  if (lane == 0) s_loss[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) t += s_loss[q];
    loss_part[blockIdx.x] = t;
  }
}

inline int grid_for(int64_t N) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((N + kWaves - 1) / kWaves, 1024)));
}

template <typename Tl, typename Td>
int launch(const void* logits, const int64_t* labels, void* dl, float* loss_part, int* bad, int64_t N, int V,
           float scale, hipStream_t st) {
  const int grid = grid_for(N);
  const Tl* lg = static_cast<const Tl*>(logits);
  Td* d = static_cast<Td*>(dl);
  const int steps = (V + 255) / 256;
  switch (steps) {
    case 1: hipLaunchKernelGGL((ce_kernel<Tl, Td, 1>), dim3(grid), dim3(kThreads), 0, st, lg, labels, d, loss_part, bad, N, V, scale); break;
    case 2: hipLaunchKernelGGL((ce_kernel<Tl, Td, 2>), dim3(grid), dim3(kThreads), 0, st, lg, labels, d, loss_part, bad, N, V, scale); break;
    case 3:
    case 4: hipLaunchKernelGGL((ce_kernel<Tl, Td, 4>), dim3(grid), dim3(kThreads), 0, st, lg, labels, d, loss_part, bad, N, V, scale); break;
    default: return fail(MG_ERR_ARG, "mg_cross_entropy_fwd_bwd: V=%d unsupported (V <= 1024)", V);
  }
  return check_launch("mg_cross_entropy_fwd_bwd");
}

}  // namespace ce
}  // namespace mg

using namespace mg;

extern "C" int mg_cross_entropy_partials(int64_t N) { return ce::grid_for(N); }

extern "C" int mg_cross_entropy_fwd_bwd(int logits_dtype, const void* logits, const int64_t* labels,
                                        int dlogits_dtype, void* dlogits, float* loss_part, int* bad_label,
                                        int64_t N, int V, float scale, void* stream) {
  const char* fn = "mg_cross_entropy_fwd_bwd";
  if (N < 1 || V < 4 || V % 4) return fail(MG_ERR_ARG, "%s: bad shape N=%lld V=%d (V %% 4 == 0)", fn, (long long)N, V);
  if (!logits || !labels || !dlogits || !loss_part) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (!aligned(logits, logits_dtype == MG_F32 ? 16 : 8) || !aligned(dlogits, dlogits_dtype == MG_F32 ? 16 : 8) ||
      !aligned(labels, 8))
    return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool lf = logits_dtype == MG_F32, lb = logits_dtype == MG_BF16;
  const bool df = dlogits_dtype == MG_F32, db = dlogits_dtype == MG_BF16;
  if (lf && db) return ce::launch<float, bf16_t>(logits, labels, dlogits, loss_part, bad_label, N, V, scale, st);
  if (lf && df) return ce::launch<float, float>(logits, labels, dlogits, loss_part, bad_label, N, V, scale, st);
  if (lb && db) return ce::launch<bf16_t, bf16_t>(logits, labels, dlogits, loss_part, bad_label, N, V, scale, st);
  if (lb && df) return ce::launch<bf16_t, float>(logits, labels, dlogits, loss_part, bad_label, N, V, scale, st);
  return fail(MG_ERR_DTYPE, "%s: dtypes (logits %d, dlogits %d) unsupported", fn, logits_dtype, dlogits_dtype);
}
