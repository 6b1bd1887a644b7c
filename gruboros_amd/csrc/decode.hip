// One-token decode step of minLM for small batches (B <= 8), bf16 weights,
// fp32 residual stream and scan state: the generation loop of reference
// generate.py:199-212, which calls minLM.forward on one token with the
// previous hiddens (reference mingru/minLM.py:97-138; minGRU's one-step
// path mingru/minGRU.py:45-52, to_out mingru/minGRU.py:41,71).
//
// Per layer two launches (three with to_out), plus one for the head:
//   mg_decode_mingru  x_in (+ pending) -> RMSNorm -> [hidden | gate] rows of
//                     to_hidden_and_gate -> one recurrence step per channel
//                     (state updated in place) -> x_out = x_in + pending + h
//                     (expansion 1), or h -> h_out as bf16 (expansion != 1)
//   mg_decode_to_out  h_out -> to_out rows -> x_out = x_in + pending + h W^T
//   mg_decode_ff      RMSNorm(x) -> Linear + GELU (-> act) ; act -> Linear
//                     -> pending (the FeedForward branch, added by the next
//                     layer's mg_decode_mingru or by the head)
//   mg_decode_head    x + pending -> RMSNorm -> to_logits
// Each workgroup recomputes the RMSNorm of the B input rows (a few KiB) into
// LDS as the bf16 vector the projection reads (or copies the B bf16 input
// rows there), then each wave produces R output rows for all B inputs: lanes
// stride the reduction dimension in 16-byte weight vectors, so the weights
// are read once, coalesced, and every weight element is used for all B rows.
// The step is weight-bandwidth bound (about 2 bytes per parameter per token);
// the launches are what a HIP graph captures.
//
// Rounding follows the bf16 training path: the norm output, the projection
// outputs, GELU's input and output and the FeedForward output are bf16
// values; the residual stream and the scan state are fp32, and the scan
// output joins the residual stream unrounded (expansion 1) or reaches to_out
// as bf16, whose fp32 sum joins it unrounded.
//
// The *_f32 entry points run the same kernels for a model kept in fp32
// (reference generate.py:277 --use-f32): fp32 weights, biases and branch
// outputs, no rounding point; each lane then reads 32 bytes of a weight row
// per 8 elements, and the staged input rows take twice the LDS (at batch 5-8
// the staged rows are at most 4096 long).

#include <algorithm>
#include <type_traits>

#include "mg_common.h"

namespace mg {
namespace decode {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16_t;  // fp16 element (a model cast with .to(torch.float16))

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxB = 8;
constexpr int kMaxStaged = 8192;  // longest bf16 input row a workgroup stages in LDS

enum Mode { MINGRU = 0, FF1 = 1, FF2 = 2, HEAD = 3, TO_OUT = 4 };

// Element type of a decode path (weights, biases, staged rows, branch outputs):
// round (the rounding point), get/put one element, load4/store4 four.
template <typename T> struct Elem;
template <> struct Elem<bf16_t> {
  static constexpr int kVec = 1;  // uint4 per 8 elements
  __device__ __forceinline__ static float round(float x) { return bf16_to_f32(f32_to_bf16(x)); }
  __device__ __forceinline__ static float get(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
  __device__ __forceinline__ static void put(bf16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
  __device__ __forceinline__ static f4 load4(const bf16_t* p) { return io4<bf16_t>::load(p); }
  __device__ __forceinline__ static void store4(bf16_t* p, const f4& v) { io4<bf16_t>::store(p, v); }
};
template <> struct Elem<float> {
  static constexpr int kVec = 2;
  __device__ __forceinline__ static float round(float x) { return x; }
  __device__ __forceinline__ static float get(const float* p, int64_t i) { return p[i]; }
  __device__ __forceinline__ static void put(float* p, int64_t i, float v) { p[i] = v; }
  __device__ __forceinline__ static f4 load4(const float* p) { return io4<float>::load(p); }
  __device__ __forceinline__ static void store4(float* p, const f4& v) { io4<float>::store(p, v); }
};
template <> struct Elem<f16_t> {
  static constexpr int kVec = 1;
  __device__ __forceinline__ static float round(float x) { return static_cast<float>(static_cast<f16_t>(x)); }
  __device__ __forceinline__ static float get(const f16_t* p, int64_t i) { return static_cast<float>(p[i]); }
  __device__ __forceinline__ static void put(f16_t* p, int64_t i, float v) { p[i] = static_cast<f16_t>(v); }
  __device__ __forceinline__ static f4 load4(const f16_t* p) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    const f16x4 x = *reinterpret_cast<const f16x4*>(p);
    f4 r;
    r.v[0] = static_cast<float>(x[0]); r.v[1] = static_cast<float>(x[1]);
    r.v[2] = static_cast<float>(x[2]); r.v[3] = static_cast<float>(x[3]);
    return r;
  }
  __device__ __forceinline__ static void store4(f16_t* p, const f4& v) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    const f16x4 x = {static_cast<f16_t>(v.v[0]), static_cast<f16_t>(v.v[1]), static_cast<f16_t>(v.v[2]),
                     static_cast<f16_t>(v.v[3])};
    *reinterpret_cast<f16x4*>(p) = x;
  }
};
// 8 consecutive elements of a row
template <typename T> struct Vec8 {
  uint4 q[Elem<T>::kVec];
};

struct Args {
  int B, D, K, rows;             // batch, model dim, reduction length, output rows
  int Di;                        // MINGRU: scan channels (rows Di .. 2 Di - 1 are the gates)
  int V;                         // embedding rows (tokens are clamped into [0, V))
  const int64_t* tokens;         // MINGRU of layer 0: x_in rows are emb[tokens[b]]
  const float* emb;              // [V, D]
  const float* x_in;             // [B, D] fp32 residual stream
  const void* pending;           // [B, D] branch output (element type) to add first (nullable)
  float* x_out;                  // MINGRU: x_in + pending + h
  const float* norm_w;           // [D]
  const void* W;                 // [rows, K]
  const void* bias;              // [rows] (nullable)
  float* state;                  // MINGRU: [B, Di] fp32 recurrence state, in place
  void* h_out;                   // MINGRU with to_out: the step's output h [B, Di] (else null)
  const void* act;               // FF2: [B, K] input; TO_OUT: h [B, Di]
  void* out;                     // FF1: act [B, F]; FF2: pending [B, D]; HEAD: logits [B, V]
  float eps;
};

// Sum each of a lane's N values over the wave (N a power of two <= 64) with
// log2(N) halving exchanges plus a butterfly: at the exchange with lane ^ o
// a lane keeps the upper half of its n live values if its bit o is set, the
// lower half otherwise, and adds its partner's copy of that half. Lane l ends
// with the total of value (l >> (6 - log2 N)); 64 / N lanes hold each total.
// (Stages are template-unrolled so every array index is a constant: a
// runtime index would turn into compare/select chains over the registers.)
// The partner of the exchange at bit o only has to differ from the lane in
// bit o and agree in the bits above it: o = 32, 16 use lane ^ o (through
// LDS's permute network), o = 8, 4, 2, 1 register-speed DPP moves within a
// row of 16 lanes: lane ^ 15 (row mirror), lane ^ 7 (half-row mirror),
// lane ^ 2 and lane ^ 1 (quad permutes). The partners across all stages
// still span every lane, so each total covers the whole wave.
template <int o>
__device__ __forceinline__ float partner(float x) {
  if constexpr (o >= 16) {
    return __shfl_xor(x, o, 64);
  } else {
    constexpr int ctrl = o == 8 ? 0x140 : o == 4 ? 0x141 : o == 2 ? 0x4E : 0xB1;  // mirror, half mirror, [2301], [1032]
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false));
  }
}

template <int n, int o, int N>
__device__ __forceinline__ void wave_sum_stage(float (&v)[N], int lane) {
  if constexpr (o >= 1) {
    if constexpr (n > 1) {
      const bool up = lane & o;
#pragma unroll
      for (int i = 0; i < n / 2; ++i) {
        const float lo = v[i], hi = v[i + n / 2];
        v[i] = (up ? hi : lo) + partner<o>(up ? lo : hi);
      }
      wave_sum_stage<n / 2, o / 2, N>(v, lane);
    } else {
      v[0] += partner<o>(v[0]);
      wave_sum_stage<1, o / 2, N>(v, lane);
    }
  }
}

template <int N>
__device__ __forceinline__ float wave_sum_n(float (&v)[N]) {
  wave_sum_stage<N, 32, N>(v, threadIdx.x & 63);
  return v[0];
}

// Where the residual-stream rows come from (a template parameter, so the
// loads carry no branches and can all be in flight together).
enum Src { SRC_X = 0, SRC_X_PENDING = 1, SRC_TOKENS = 2 };

// Residual-stream value (b, c) before the norm: x_in (or the embedding row)
// plus the pending branch output.
template <typename T, int SRC>
__device__ __forceinline__ float stream_at(const Args& a, int b, int c) {
  float x;
  if constexpr (SRC == SRC_TOKENS) {
    const int64_t t = min(max(a.tokens[b], int64_t(0)), static_cast<int64_t>(a.V - 1));
    x = a.emb[t * a.D + c];
  } else {
    x = a.x_in[static_cast<int64_t>(b) * a.D + c];
  }
  if constexpr (SRC == SRC_X_PENDING) x += Elem<T>::get(static_cast<const T*>(a.pending), static_cast<int64_t>(b) * a.D + c);
  return x;
}

// The same for columns c .. c + 3 (c a multiple of 4; rows are 16-byte aligned).
template <typename T, int SRC>
__device__ __forceinline__ f4 stream4_at(const Args& a, int b, int c) {
  f4 x;
  if constexpr (SRC == SRC_TOKENS) {
    const int64_t t = min(max(a.tokens[b], int64_t(0)), static_cast<int64_t>(a.V - 1));
    x = io4<float>::load(a.emb + t * a.D + c);
  } else {
    x = io4<float>::load(a.x_in + static_cast<int64_t>(b) * a.D + c);
  }
  if constexpr (SRC == SRC_X_PENDING) {
    const f4 p = Elem<T>::load4(static_cast<const T*>(a.pending) + static_cast<int64_t>(b) * a.D + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) x.v[e] += p.v[e];
  }
  return x;
}

// MODE: which step; BP: batch rows (padded); R: output rows per wave;
// NC: 512-element chunks of the reduction a lane covers (K <= 512 NC); CPT:
// columns per thread in the norm prologue (D <= 256 CPT; a multiple of 4, or
// 1 where there is no norm). The input rows are staged in a static LDS array
// of BP x 512 NC bf16 values (at most 8 x 8192 = 128 KiB, within gfx950's
// 160 KiB per workgroup).
template <typename T, int MODE, int SRC, int BP, int R, int NC, int CPT>
__global__ __launch_bounds__(kThreads) void decode_kernel(Args a) {
  static_assert(NC * 512 <= kMaxStaged, "staged row length");
  constexpr bool kStagedInput = MODE == FF2 || MODE == TO_OUT;  // input rows as they are, no norm
  constexpr int kV = Elem<T>::kVec;
  __shared__ uint4 lds[BP * NC * 64 * kV];
  T* s_in = reinterpret_cast<T*>(lds);  // [BP][K]
  const T* W = static_cast<const T*>(a.W);
  __shared__ float s_part[kWaves][BP];
  __shared__ float s_rstd[BP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = a.K;

  // 0. this wave's weight rows (MINGRU: rows d and D+d, hidden and gate of
  // channel d), requested before anything else so that their latency
  // overlaps the norm prologue
  const int g = blockIdx.x * kWaves + wave;  // row group
  int rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rows[r] = MODE == MINGRU ? g + r * a.Di : g * R + r;
  const bool active = rows[0] < (MODE == MINGRU ? a.Di : a.rows);
  Vec8<T> wv[NC][R];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // clamped, unconditional loads (nothing branches between them); rows
      // past the end are never used, chunks past K are skipped below
      const int k0 = min(c * 512 + lane * 8, K - 8);
      const int row = active ? rows[r] : 0;
#pragma unroll
      for (int j = 0; j < kV; ++j)
        wv[c][r].q[j] = reinterpret_cast<const uint4*>(W + static_cast<int64_t>(row) * K + k0)[j];
    }

  // 1. the B input rows, as bf16, into LDS (rows B..BP-1 zero)
  if constexpr (kStagedInput) {
    // kBatch 16-byte loads per thread in flight before their LDS stores (a
    // load-store pair per iteration would wait out one memory latency each)
    constexpr int kBatch = 8;
    constexpr int kPer16 = 16 / static_cast<int>(sizeof(T));  // elements per 16 bytes
    const int n16 = BP * (K / kPer16);
    const T* act = static_cast<const T*>(a.act);
    for (int i0 = 0; i0 < n16; i0 += kBatch * kThreads) {
      uint4 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = i0 + u * kThreads + tid;
        const int b = i / (K / kPer16), c16 = i % (K / kPer16);
        v[u] = make_uint4(0, 0, 0, 0);
        if (i < n16 && b < a.B)
          v[u] = *reinterpret_cast<const uint4*>(act + static_cast<int64_t>(b) * K + c16 * kPer16);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = i0 + u * kThreads + tid;
        if (i < n16) reinterpret_cast<uint4*>(s_in)[i] = v[u];
      }
    }
  } else {
    // RMSNorm over D = K: the rows are read once into registers (columns
    // 4 (tid + 256 q) .. +3 in one 16-byte load per row and q), the sum of
    // squares reduced over the workgroup, then y = x r w goes to LDS
    static_assert(CPT % 4 == 0, "whole 4-column groups per thread");
    constexpr int Q = CPT / 4;
    float xr[BP][CPT];
    float ss[BP];
#pragma unroll
    for (int b = 0; b < BP; ++b) {
      ss[b] = 0.0f;
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const int c = 4 * (tid + q * kThreads);
        const f4 x = stream4_at<T, SRC>(a, min(b, a.B - 1), min(c, K - 4));  // unconditional load
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xr[b][4 * q + e] = (b < a.B && c < K) ? x.v[e] : 0.0f;
          ss[b] += xr[b][4 * q + e] * xr[b][4 * q + e];
        }
      }
    }
    {
      // lane l ends with the wave's total of row l / (64 / BP)
      const float s = wave_sum_n<BP>(ss);
      if (lane % (64 / BP) == 0) s_part[wave][lane / (64 / BP)] = s;
    }
    __syncthreads();
    if (tid < BP) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += s_part[w][tid];
      s_rstd[tid] = __builtin_amdgcn_rsqf(s / static_cast<float>(K) + a.eps);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int c = 4 * (tid + q * kThreads);
      if (c < K) {
        const f4 w = io4<float>::load(a.norm_w + c);
#pragma unroll
        for (int b = 0; b < BP; ++b) {
          f4 y;
#pragma unroll
          for (int e = 0; e < 4; ++e) y.v[e] = xr[b][4 * q + e] * s_rstd[b] * w.v[e];
          Elem<T>::store4(s_in + b * K + c, y);
        }
      }
    }
  }
  __syncthreads();
  if (!active) return;

  // 2. the dot products, weights from registers, inputs from LDS
  float acc[R][BP];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < BP; ++b) acc[r][b] = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k0 = c * 512 + lane * 8;
    if (k0 >= K) break;
#pragma unroll
    for (int b = 0; b < BP; ++b) {
      if constexpr (kV == 1) {
        const uint4 xv = *reinterpret_cast<const uint4*>(s_in + b * K + k0);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint4 wq = wv[c][r].q[0];
          const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {  // two 16-bit products per instruction, fp32 accumulation
            if constexpr (sizeof(T) == 2 && !std::is_same<T, f16_t>::value)
              acc[r][b] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, ww[q]),
                                                          __builtin_bit_cast(bf16x2, xw[q]), acc[r][b], false);
            else
              acc[r][b] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, ww[q]), __builtin_bit_cast(f16x2, xw[q]),
                                                 acc[r][b], false);
          }
        }
      } else {
        const float4 x0 = reinterpret_cast<const float4*>(s_in + b * K + k0)[0];
        const float4 x1 = reinterpret_cast<const float4*>(s_in + b * K + k0)[1];
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint4 w0 = wv[c][r].q[0], w1 = wv[c][r].q[1];
          const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r][b] = __builtin_fmaf(__uint_as_float(ww[e]), xs[e], acc[r][b]);
        }
      }
    }
  }
  constexpr int N = R * BP;
  float flat[N];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < BP; ++b) flat[r * BP + b] = acc[r][b];
  const float sum = wave_sum_n<N>(flat);

  // 3. epilogue: the first lane holding value (r, b) = (idx / BP, idx % BP)
  constexpr int kCopies = 64 / N;
  const int idx = lane / kCopies, r = idx / BP, b = idx % BP;
  if (MODE == MINGRU) {
    // hidden (r = 0) and gate (r = 1) of one batch row are 32 lanes apart
    const float other = __shfl_xor(sum, 32, 64);
    if (lane % kCopies || r != 0 || b >= a.B) return;
    const int d = g;
    const float hid = Elem<T>::round(sum), gate = Elem<T>::round(other);
    float coef, v;
    fwd_coeffs(gate, hid, coef, v);
    float* st = a.state + static_cast<int64_t>(b) * a.Di + d;
    const float h = coef * *st + v;
    *st = h;
    if (a.h_out) Elem<T>::put(static_cast<T*>(a.h_out), static_cast<int64_t>(b) * a.Di + d, h);
    else a.x_out[static_cast<int64_t>(b) * a.D + d] = stream_at<T, SRC>(a, b, d) + h;
    return;
  }
  if (lane % kCopies || b >= a.B) return;
  if constexpr (MODE == TO_OUT) {
    const int d = rows[0] + r;
    a.x_out[static_cast<int64_t>(b) * a.D + d] = stream_at<T, SRC>(a, b, d) + sum;
    return;
  }
  T* o = static_cast<T*>(a.out);
  const int64_t oi = static_cast<int64_t>(b) * a.rows + rows[0] + r;
  if constexpr (MODE == FF1) {
    Elem<T>::put(o, oi, gelu(Elem<T>::round(sum + Elem<T>::get(static_cast<const T*>(a.bias), rows[0] + r))));
  } else if constexpr (MODE == FF2) {
    Elem<T>::put(o, oi, sum + Elem<T>::get(static_cast<const T*>(a.bias), rows[0] + r));
  } else {
    Elem<T>::put(o, oi, sum);
  }
}

// The staged-input modes (FF2, TO_OUT) take K <= 8192 (NC 8 up to 4096, else
// 16); the norm modes K = D <= 2048 (NC 2 up to 1024, else 4). Every wave's
// lane covers its chunks with K <= 512 NC, which check_shape guarantees. fp32
// rows take twice the LDS, so at batch 5-8 an fp32 staged row is at most 4096
// long (the 16-chunk variant is not built there).
template <typename T, int MODE, int SRC, int BP, int R>
int launch_bp(const Args& a, dim3 grid, hipStream_t st) {
  if constexpr (MODE == FF2 || MODE == TO_OUT) {
    if (a.K <= 4096) {
      hipLaunchKernelGGL((decode_kernel<T, MODE, SRC, BP, R, 8, 1>), grid, dim3(kThreads), 0, st, a);
    } else {
      if constexpr (sizeof(T) == 4 && BP == 8)
        return fail(MG_ERR_ARG, "mg_decode: fp32 staged rows of %d > 4096 at batch %d", a.K, a.B);
      else
        hipLaunchKernelGGL((decode_kernel<T, MODE, SRC, BP, R, 16, 1>), grid, dim3(kThreads), 0, st, a);
    }
  } else {
    if (a.K <= 1024) hipLaunchKernelGGL((decode_kernel<T, MODE, SRC, BP, R, 2, 4>), grid, dim3(kThreads), 0, st, a);
    else hipLaunchKernelGGL((decode_kernel<T, MODE, SRC, BP, R, 4, 8>), grid, dim3(kThreads), 0, st, a);
  }
  return check_launch("mg_decode");
}

template <typename T, int MODE, int SRC, int R>
int launch(const Args& a, hipStream_t st) {
  const int groups = MODE == MINGRU ? a.Di : a.rows / R;
  const dim3 grid((groups + kWaves - 1) / kWaves);
  const int BP = a.B <= 1 ? 1 : a.B <= 2 ? 2 : a.B <= 4 ? 4 : 8;
  switch (BP) {
    case 1: return launch_bp<T, MODE, SRC, 1, R>(a, grid, st);
    case 2: return launch_bp<T, MODE, SRC, 2, R>(a, grid, st);
    case 4: return launch_bp<T, MODE, SRC, 4, R>(a, grid, st);
    default: return launch_bp<T, MODE, SRC, 8, R>(a, grid, st);
  }
}

// kmax: 2048 for the model dimension (norm prologue), 8192 for a staged input
// row (the FeedForward width, to_out's Di); fp32 staged rows at batch 5-8: 4096
inline int check_shape(const char* fn, int B, int K, int kmax) {
  if (B < 1 || B > kMaxB) return fail(MG_ERR_ARG, "%s: batch %d outside [1, %d]", fn, B, kMaxB);
  if (K < 8 || K % 8 || K > kmax)
    return fail(MG_ERR_ARG, "%s: length %d must be a positive multiple of 8, at most %d", fn, K, kmax);
  return MG_OK;
}
template <typename T>
int staged_max(int B) {
  return sizeof(T) == 4 && B > 4 ? 4096 : kMaxStaged;
}

// Alignment of the element-type vectors read 16 (weights, staged rows) or 4
// elements (pending) at a time.
template <typename T>
constexpr size_t kPendAlign = 4 * sizeof(T);

template <typename T>
int mingru_impl(const char* fn, int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                const float* x_in, const void* pending, float* x_out, void* h_out, const float* norm_w,
                const void* w_hg, float* state, float eps, void* stream) {
  if (int rc = check_shape(fn, B, D, 2048)) return rc;
  if (h_out)
    if (int rc = check_shape(fn, B, Di, staged_max<T>(B))) return rc;
  if (!(tokens ? (emb != nullptr && V >= 1) : x_in != nullptr) || !(h_out || x_out) || !norm_w || !w_hg || !state)
    return fail(MG_ERR_ARG, "%s: NULL pointer or empty embedding", fn);
  if (!aligned(w_hg, 16) || !aligned(norm_w, 16) || (tokens ? !aligned(emb, 16) : !aligned(x_in, 16)) ||
      (pending && !aligned(pending, kPendAlign<T>)))
    return fail(MG_ERR_ARG, "%s: weight, norm weight, emb or x_in not 16-byte aligned, or pending not %zu-byte aligned",
                fn, kPendAlign<T>);
  Args a{};
  a.B = B; a.D = D; a.Di = Di; a.K = D; a.rows = 2 * Di; a.V = V;
  a.tokens = tokens; a.emb = emb; a.x_in = x_in; a.pending = pending;
  a.x_out = x_out; a.h_out = h_out; a.norm_w = norm_w; a.W = w_hg; a.state = state; a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (tokens) return launch<T, MINGRU, SRC_TOKENS, 2>(a, st);
  if (pending) return launch<T, MINGRU, SRC_X_PENDING, 2>(a, st);
  return launch<T, MINGRU, SRC_X, 2>(a, st);
}

template <typename T>
int to_out_impl(const char* fn, int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                const float* x_in, const void* pending, const void* h, const void* w_out, float* x_out,
                void* stream) {
  if (int rc = check_shape(fn, B, D, 2048)) return rc;
  if (int rc = check_shape(fn, B, Di, staged_max<T>(B))) return rc;
  if (!(tokens ? (emb != nullptr && V >= 1) : x_in != nullptr) || !h || !w_out || !x_out)
    return fail(MG_ERR_ARG, "%s: NULL pointer or empty embedding", fn);
  if (!aligned(w_out, 16) || !aligned(h, 16) || (tokens ? !aligned(emb, 16) : !aligned(x_in, 16)) ||
      (pending && !aligned(pending, kPendAlign<T>)))
    return fail(MG_ERR_ARG, "%s: weight, h, emb or x_in not 16-byte aligned, or pending not %zu-byte aligned", fn,
                kPendAlign<T>);
  Args a{};
  a.B = B; a.D = D; a.Di = Di; a.K = Di; a.rows = D; a.V = V;
  a.tokens = tokens; a.emb = emb; a.x_in = x_in; a.pending = pending;
  a.act = h; a.W = w_out; a.x_out = x_out;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (tokens) return launch<T, TO_OUT, SRC_TOKENS, 1>(a, st);
  if (pending) return launch<T, TO_OUT, SRC_X_PENDING, 1>(a, st);
  return launch<T, TO_OUT, SRC_X, 1>(a, st);
}

template <typename T>
int ff_impl(const char* fn, int B, int D, int F, const float* x, const float* norm_w, const void* w1, const void* b1,
            void* act, const void* w2, const void* b2, void* pending_out, float eps, void* stream) {
  if (int rc = check_shape(fn, B, D, 2048)) return rc;
  if (int rc = check_shape(fn, B, F, staged_max<T>(B))) return rc;
  if (!x || !norm_w || !w1 || !b1 || !act || !w2 || !b2 || !pending_out) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (F % 4 || !aligned(w1, 16) || !aligned(w2, 16) || !aligned(act, 16) || !aligned(x, 16) || !aligned(norm_w, 16))
    return fail(MG_ERR_ARG, "%s: F %% 4, 16-byte weights, act, x and norm weight required", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  Args a{};
  a.B = B; a.D = D; a.K = D; a.rows = F;
  a.x_in = x; a.norm_w = norm_w; a.W = w1; a.bias = b1; a.out = act; a.eps = eps;
  if (int rc = launch<T, FF1, SRC_X, 4>(a, st)) return rc;
  Args c{};
  c.B = B; c.D = D; c.K = F; c.rows = D;
  c.act = act; c.W = w2; c.bias = b2; c.out = pending_out;
  return launch<T, FF2, SRC_X, 1>(c, st);
}

template <typename T>
int head_impl(const char* fn, int B, int D, int V, const float* x_in, const void* pending, const float* norm_w,
              const void* w_out, void* logits, float eps, void* stream) {
  if (int rc = check_shape(fn, B, D, 2048)) return rc;
  if (V < 1 || !x_in || !norm_w || !w_out || !logits) return fail(MG_ERR_ARG, "%s: bad argument", fn);
  if (!aligned(w_out, 16) || !aligned(x_in, 16) || !aligned(norm_w, 16) || (pending && !aligned(pending, kPendAlign<T>)))
    return fail(MG_ERR_ARG, "%s: weight, x_in or norm weight not 16-byte aligned, or pending not %zu-byte aligned", fn,
                kPendAlign<T>);
  Args a{};
  a.B = B; a.D = D; a.K = D; a.rows = V;
  a.x_in = x_in; a.pending = pending; a.norm_w = norm_w; a.W = w_out; a.out = logits; a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (pending) return launch<T, HEAD, SRC_X_PENDING, 1>(a, st);
  return launch<T, HEAD, SRC_X, 1>(a, st);
}

}  // namespace decode
}  // namespace mg

using namespace mg;

extern "C" int mg_decode_mingru(int B, int D, const int64_t* tokens, const float* emb, int V, const float* x_in,
                                const void* pending, float* x_out, const float* norm_w, const void* w_hg,
                                float* state, float eps, void* stream) {
  if (!x_out) return fail(MG_ERR_ARG, "mg_decode_mingru: x_out is NULL");
  return decode::mingru_impl<bf16_t>("mg_decode_mingru", B, D, D, tokens, emb, V, x_in, pending, x_out, nullptr,
                                     norm_w, w_hg, state, eps, stream);
}

extern "C" int mg_decode_mingru_expanded(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                                         const float* x_in, const void* pending, void* h_out, const float* norm_w,
                                         const void* w_hg, float* state, float eps, void* stream) {
  if (!h_out) return fail(MG_ERR_ARG, "mg_decode_mingru_expanded: h_out is NULL");
  return decode::mingru_impl<bf16_t>("mg_decode_mingru_expanded", B, D, Di, tokens, emb, V, x_in, pending, nullptr,
                                     h_out, norm_w, w_hg, state, eps, stream);
}

extern "C" int mg_decode_to_out(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                                const float* x_in, const void* pending, const void* h, const void* w_out,
                                float* x_out, void* stream) {
  return decode::to_out_impl<bf16_t>("mg_decode_to_out", B, D, Di, tokens, emb, V, x_in, pending, h, w_out, x_out,
                                     stream);
}

extern "C" int mg_decode_ff(int B, int D, int F, const float* x, const float* norm_w, const void* w1,
                            const void* b1, void* act, const void* w2, const void* b2, void* pending_out, float eps,
                            void* stream) {
  return decode::ff_impl<bf16_t>("mg_decode_ff", B, D, F, x, norm_w, w1, b1, act, w2, b2, pending_out, eps, stream);
}

extern "C" int mg_decode_head(int B, int D, int V, const float* x_in, const void* pending, const float* norm_w,
                              const void* w_out, void* logits, float eps, void* stream) {
  return decode::head_impl<bf16_t>("mg_decode_head", B, D, V, x_in, pending, norm_w, w_out, logits, eps, stream);
}

// fp32 models (reference generate.py --use-f32): the same steps over fp32
// weights, biases, branch outputs and logits.
extern "C" int mg_decode_mingru_f32(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                                    const float* x_in, const float* pending, float* x_out, float* h_out,
                                    const float* norm_w, const float* w_hg, float* state, float eps, void* stream) {
  if (!x_out == !h_out) return fail(MG_ERR_ARG, "mg_decode_mingru_f32: exactly one of x_out and h_out");
  if (!h_out && Di != D) return fail(MG_ERR_ARG, "mg_decode_mingru_f32: Di %d != D %d needs h_out", Di, D);
  return decode::mingru_impl<float>("mg_decode_mingru_f32", B, D, Di, tokens, emb, V, x_in, pending, x_out, h_out,
                                    norm_w, w_hg, state, eps, stream);
}

extern "C" int mg_decode_to_out_f32(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                                    const float* x_in, const float* pending, const float* h, const float* w_out,
                                    float* x_out, void* stream) {
  return decode::to_out_impl<float>("mg_decode_to_out_f32", B, D, Di, tokens, emb, V, x_in, pending, h, w_out, x_out,
                                    stream);
}

extern "C" int mg_decode_ff_f32(int B, int D, int F, const float* x, const float* norm_w, const float* w1,
                                const float* b1, float* act, const float* w2, const float* b2, float* pending_out,
                                float eps, void* stream) {
  return decode::ff_impl<float>("mg_decode_ff_f32", B, D, F, x, norm_w, w1, b1, act, w2, b2, pending_out, eps,
                                stream);
}

extern "C" int mg_decode_head_f32(int B, int D, int V, const float* x_in, const float* pending, const float* norm_w,
                                  const float* w_out, float* logits, float eps, void* stream) {
  return decode::head_impl<float>("mg_decode_head_f32", B, D, V, x_in, pending, norm_w, w_out, logits, eps, stream);
}

// fp16 models (reference generate.py:143-144, --use-fp16 with --use-f32): the
// bf16 steps with fp16 weights and fp16 rounding points.
extern "C" int mg_decode_mingru_f16(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                                    const float* x_in, const void* pending, float* x_out, void* h_out,
                                    const float* norm_w, const void* w_hg, float* state, float eps, void* stream) {
  if (!x_out == !h_out) return fail(MG_ERR_ARG, "mg_decode_mingru_f16: exactly one of x_out and h_out");
  if (!h_out && Di != D) return fail(MG_ERR_ARG, "mg_decode_mingru_f16: Di %d != D %d needs h_out", Di, D);
  return decode::mingru_impl<decode::f16_t>("mg_decode_mingru_f16", B, D, Di, tokens, emb, V, x_in, pending, x_out,
                                            h_out, norm_w, w_hg, state, eps, stream);
}

extern "C" int mg_decode_to_out_f16(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                                    const float* x_in, const void* pending, const void* h, const void* w_out,
                                    float* x_out, void* stream) {
  return decode::to_out_impl<decode::f16_t>("mg_decode_to_out_f16", B, D, Di, tokens, emb, V, x_in, pending, h, w_out,
                                            x_out, stream);
}

extern "C" int mg_decode_ff_f16(int B, int D, int F, const float* x, const float* norm_w, const void* w1,
                                const void* b1, void* act, const void* w2, const void* b2, void* pending_out,
                                float eps, void* stream) {
  return decode::ff_impl<decode::f16_t>("mg_decode_ff_f16", B, D, F, x, norm_w, w1, b1, act, w2, b2, pending_out, eps,
                                        stream);
}

extern "C" int mg_decode_head_f16(int B, int D, int V, const float* x_in, const void* pending, const float* norm_w,
                                  const void* w_out, void* logits, float eps, void* stream) {
  return decode::head_impl<decode::f16_t>("mg_decode_head_f16", B, D, V, x_in, pending, norm_w, w_out, logits, eps,
                                          stream);
}
