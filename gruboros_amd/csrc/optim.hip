// Schedule-Free AdamW parameter update, all parameter tensors in one launch.
//
// Reference: the training loop steps schedulefree.AdamWScheduleFree
// (train.py:635 construction, :642 train mode, :808 step; package pinned at
// requirements.txt:44). The per-element update restates the published
// algorithm (Defazio et al. 2024) in the package's train-mode form, with y
// the parameter, z the base iterate and v the second moment:
//   v <- b2 v + (1 - b2) g^2
//   u  = g / (sqrt(v / bc2) + eps) + wd y          (y before this step)
//   y <- (1 - c) y + c z + y_lr u                  (c = ckp1)
//   z <- z - lr u
// Optionally also writes y rounded to bf16 (the weights the next forward's
// bf16 GEMMs read), so no separate cast pass is needed.
//
// Memory: 16 bytes read + 12 (+2) written per parameter, one pass.

#include <algorithm>

#include "mg_common.h"

namespace mg {
namespace sf {

constexpr int kThreads = 256;
constexpr int kChunk = kThreads * 4 * 8;  // elements per workgroup: 8 float4 per thread

// Must match mg_sf_tensor in include/mingru_hip.h.
struct Tensor {
  float* p;
  const float* g;
  float* z;
  float* v;
  bf16_t* p_bf16;
  int64_t n;
  int64_t chunk_start;  // first chunk index of this tensor
  int64_t pair_cols;    // > 0: p_bf16 is the hi/lo pair of p viewed as [n / pair_cols, pair_cols]
};

struct Hyper {
  float b2, one_minus_b2, inv_bc2, eps, wd, ckp1, y_lr, lr;
};

__device__ __forceinline__ void update(float& y, float g, float& z, float& v, const Hyper& h) {
  v = h.b2 * v + h.one_minus_b2 * g * g;
  const float u = g / (sqrtf(v * h.inv_bc2) + h.eps) + h.wd * y;
  y = (1.0f - h.ckp1) * y + h.ckp1 * z + h.y_lr * u;
  z = z - h.lr * u;
}

// The fp32 state streams (parameter, gradient, z, v: 2.4 GB a step at cfg3,
// each touched once) load and store with the non-temporal hint: measured
// 504 -> 441 us a step at cfg3. The bf16 copies keep plain stores (with the
// hint they measured slower: the next step's products read them).
typedef float f32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4 load4_stream(const float* q) {
  const f32x4_nt x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(q));
  f4 r;
  r.v[0] = x[0]; r.v[1] = x[1]; r.v[2] = x[2]; r.v[3] = x[3];
  return r;
}
__device__ __forceinline__ void store4_stream(float* q, const f4& r) {
  const f32x4_nt x = {r.v[0], r.v[1], r.v[2], r.v[3]};
  __builtin_nontemporal_store(x, reinterpret_cast<f32x4_nt*>(q));
}

__global__ __launch_bounds__(kThreads) void sf_adamw_kernel(const Tensor* __restrict__ ts, int nt, Hyper h) {
  // tensor owning this chunk: last t with chunk_start <= blockIdx.x
  int lo = 0, hi = nt - 1;
  const int64_t b = blockIdx.x;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ts[mid].chunk_start <= b) lo = mid; else hi = mid - 1;
  }
  const Tensor t = ts[lo];
  const int64_t base = (b - t.chunk_start) * kChunk;
  const bool vec = (t.n % 4) == 0;
#pragma unroll 2
  for (int r = 0; r < kChunk / (kThreads * 4); ++r) {
    const int64_t i = base + (static_cast<int64_t>(r) * kThreads + threadIdx.x) * 4;
    if (i >= t.n) break;
    if (vec) {
      f4 y = load4_stream(t.p + i), g = load4_stream(t.g + i), z = load4_stream(t.z + i), v = load4_stream(t.v + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) update(y.v[j], g.v[j], z.v[j], v.v[j], h);
      store4_stream(t.p + i, y);
      store4_stream(t.z + i, z);
      store4_stream(t.v + i, v);
      if (t.p_bf16) {
        if (t.pair_cols > 0) {  // row r = i / C: hi at r * 2C + c, lo at r * 2C + C + c (4 | C)
          const uint32_t C = static_cast<uint32_t>(t.pair_cols);
          const int64_t r = static_cast<int64_t>(static_cast<uint32_t>(i) / C);
          const int64_t c = i - r * C;
          f4 lo;
#pragma unroll
          for (int j = 0; j < 4; ++j) lo.v[j] = y.v[j] - bf16_to_f32(f32_to_bf16(y.v[j]));
          io4<bf16_t>::store(t.p_bf16 + r * 2 * C + c, y);
          io4<bf16_t>::store(t.p_bf16 + r * 2 * C + C + c, lo);
        } else {
          io4<bf16_t>::store(t.p_bf16 + i, y);
        }
      }
    } else {
      for (int64_t k = i; k < std::min<int64_t>(i + 4, t.n); ++k) {
        float y = t.p[k], z = t.z[k], v = t.v[k];
        update(y, t.g[k], z, v, h);
        t.p[k] = y;
        t.z[k] = z;
        t.v[k] = v;
        if (t.p_bf16) {
          if (t.pair_cols > 0) {
            const int64_t r = k / t.pair_cols, c = k - r * t.pair_cols;
            const bf16_t hi = f32_to_bf16(y);
            t.p_bf16[r * 2 * t.pair_cols + c] = hi;
            t.p_bf16[r * 2 * t.pair_cols + t.pair_cols + c] = f32_to_bf16(y - bf16_to_f32(hi));
          } else {
            t.p_bf16[k] = f32_to_bf16(y);
          }
        }
      }
    }
  }
}

}  // namespace sf
}  // namespace mg

using namespace mg;

extern "C" int64_t mg_sf_adamw_chunk_elems(void) { return sf::kChunk; }

extern "C" int mg_sf_adamw_step(const void* tensors, int ntensors, int64_t nchunks, float beta2,
                                float one_minus_beta2, float bias_correction2, float eps, float weight_decay,
                                float ckp1, float y_lr, float lr, void* stream) {
  const char* fn = "mg_sf_adamw_step";
  if (!tensors || ntensors < 1 || nchunks < 1 || nchunks > 0x7fffffffLL)
    return fail(MG_ERR_ARG, "%s: bad table (ntensors=%d, nchunks=%lld)", fn, ntensors, (long long)nchunks);
  if (!aligned(tensors, 8)) return fail(MG_ERR_ARG, "%s: table misaligned", fn);
  if (!(bias_correction2 > 0.0f)) return fail(MG_ERR_ARG, "%s: bias_correction2 must be > 0", fn);
  sf::Hyper h{beta2, one_minus_beta2, 1.0f / bias_correction2, eps, weight_decay, ckp1, y_lr, lr};
  hipLaunchKernelGGL(sf::sf_adamw_kernel, dim3(static_cast<unsigned>(nchunks)), dim3(sf::kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const sf::Tensor*>(tensors), ntensors, h);
  return check_launch(fn);
}
