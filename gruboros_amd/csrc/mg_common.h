// Shared device helpers and host-side error plumbing for libmingru_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include <algorithm>
#include <type_traits>

#include "mingru_hip.h"

namespace mg {

// ---------------------------------------------------------------- errors

// Per-thread message of the last failure; returned by mg_last_error().
char* last_error_buf();

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(last_error_buf(), 512, fmt, ap);
  va_end(ap);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MG_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MG_OK;
}

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---------------------------------------------------------------- bf16 / vectors

typedef unsigned short bf16_t;  // raw bfloat16 bits in memory

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

// ---------------------------------------------------------------- stochastic rounding
//
// Gradients stored in bf16 are rounded stochastically: up (in magnitude)
// with probability equal to the dropped fraction of a bf16 ulp, so the
// expected value is the fp32 value. With round-to-nearest each element's
// error is a fixed function of its value. At a nearly uniform softmax (the
// untrained model) every row of the logits gradient is (1/V - onehot)/N up
// to small deviations, so the rows of one label share one rounding error, and
// those errors add up over the rows of a weight gradient instead of
// cancelling: on the fp64 restatement at the cfg3 model size they moved the
// FeedForward and norm weight gradients by 4-7% at 8-16 k rows, growing with
// the row count; with stochastic rounding by 0.5%, independent of it.
// The random bits are a hash of the element pair's index, its values and a
// salt per call site, so the result is a deterministic function of the inputs
// (no generator state: replays and resumed runs repeat bit for bit). One
// 32-bit hash serves two elements (16 bits each), and the rounding itself is
// gfx950's v_cvt_sr_bf16_f32, which adds the HIGH 16 bits of its random
// operand below the bf16 mantissa and truncates, i.e. for finite x
// bf16(x) = (bits(x) + (r >> 16)) >> 16, and keeps Inf and NaN (checked
// against that rule on the device for 2^20 random operands).
// The hash is Knuth's multiplicative (Fibonacci) hash on 24 bits, x * 2^24/phi
// (the low 24 bits of x; bits 16-31 of the 48-bit product go to the first
// element), with one xorshift folding those high bits into the low half that
// the pair's second element uses: consecutive indices give equidistributed
// (low-discrepancy) thresholds along a row and down a column. The 24-bit
// multiply is a full-rate instruction (v_mul_u32_u24; a 32-bit multiply runs
// at a quarter of the rate), which matters where the rounding sits in an
// HBM-bound loop (the scan backward: two gradients per element).
__device__ __forceinline__ uint32_t sr_hash(uint32_t x) {
  x = __umul24(x, 0x9e3779u);
  return x ^ (x >> 15);
}

typedef __bf16 __attribute__((ext_vector_type(2))) bf16x2_t;

// (lo, hi) fp32 -> packed bf16 pair (lo in the low half), each rounded
// stochastically. idx: lo's index in its tensor (hi is idx + 1).
__device__ __forceinline__ uint32_t pack_bf16x2_sr(float lo, float hi, uint32_t idx, uint32_t salt) {
  const uint32_t r = sr_hash(idx ^ salt ^ __float_as_uint(lo) ^ __builtin_rotateleft32(__float_as_uint(hi), 16));
  bf16x2_t v = {};
  v = __builtin_amdgcn_cvt_sr_bf16_f32(v, lo, r, false);
  v = __builtin_amdgcn_cvt_sr_bf16_f32(v, hi, r << 16, true);
  return __builtin_bit_cast(uint32_t, v);
}

// Two pairs that belong together (the scan backward's dgate and dhidden of
// the same two elements) from ONE hash: the first pair takes the 16-bit
// windows r[31:16] and r[15:0], the second the windows of r rotated by 8
// bits (r[7:0]r[31:24] and r[23:8]). Each window is uniform on its own, and
// the leading byte of every window is a distinct byte of r, so the four
// roundings are unbiased and nearly independent, at half the hashes.
// idx: the first pair's index (its lo element) with the call site's salt added.
__device__ __forceinline__ void pack2_bf16x2_sr(float a0, float a1, float b0, float b1, uint32_t idx,
                                                uint32_t& pa, uint32_t& pb) {
  const uint32_t r = sr_hash(idx ^ __float_as_uint(a0));
  const uint32_t r2 = __builtin_rotateright32(r, 8);
  bf16x2_t va = __builtin_nondeterministic_value(va), vb = __builtin_nondeterministic_value(vb);
  va = __builtin_amdgcn_cvt_sr_bf16_f32(va, a0, r, false);
  va = __builtin_amdgcn_cvt_sr_bf16_f32(va, a1, r << 16, true);
  vb = __builtin_amdgcn_cvt_sr_bf16_f32(vb, b0, r2, false);
  vb = __builtin_amdgcn_cvt_sr_bf16_f32(vb, b1, r2 << 16, true);
  pa = __builtin_bit_cast(uint32_t, va);
  pb = __builtin_bit_cast(uint32_t, vb);
}

// N consecutive channels of one row, loaded/stored as one vector access
// (N = 4: 8-byte bf16 / 16-byte fp32; N = 8: 16-byte bf16 / 2 x 16-byte fp32).
template <int N>
struct fv {
  float v[N];
};
using f4 = fv<4>;

template <typename T, int N> struct iov;

template <int N> struct iov<float, N> {
  static_assert(N % 4 == 0, "fp32 vectors are multiples of float4");
  __device__ __forceinline__ static fv<N> fill(float x) {
    fv<N> r;
#pragma unroll
    for (int j = 0; j < N; ++j) r.v[j] = x;
    return r;
  }
  __device__ __forceinline__ static fv<N> load(const float* p) {
    fv<N> r;
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const float4 x = reinterpret_cast<const float4*>(p)[q];
      r.v[4 * q] = x.x; r.v[4 * q + 1] = x.y; r.v[4 * q + 2] = x.z; r.v[4 * q + 3] = x.w;
    }
    return r;
  }
  __device__ __forceinline__ static void store(float* p, const fv<N>& a) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q)
      reinterpret_cast<float4*>(p)[q] = make_float4(a.v[4 * q], a.v[4 * q + 1], a.v[4 * q + 2], a.v[4 * q + 3]);
  }
  // Streaming store (non-temporal hint): for outputs no later kernel step rereads soon.
  __device__ __forceinline__ static void store_nt(float* p, const fv<N>& a) {
#pragma unroll
    for (int j = 0; j < N; ++j) __builtin_nontemporal_store(a.v[j], p + j);
  }
  // Gradient stores (fp32: exact; the bf16 versions round stochastically).
  __device__ __forceinline__ static void store_grad(float* p, const fv<N>& a, uint32_t, uint32_t) { store(p, a); }
  __device__ __forceinline__ static void store_grad_nt(float* p, const fv<N>& a, uint32_t, uint32_t) {
    store_nt(p, a);
  }
  __device__ __forceinline__ static void store_grad2_nt(float* pa, const fv<N>& a, float* pb, const fv<N>& b,
                                                        uint32_t) {
    store_nt(pa, a);
    store_nt(pb, b);
  }
};

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

template <int N> struct iov<bf16_t, N> {
  static_assert(N == 4 || N == 8, "bf16 vectors are 8 or 16 bytes");
  using raw = typename std::conditional<N == 4, uint2, uint4>::type;
  __device__ __forceinline__ static fv<N> fill(float x) {
    const float r = bf16_to_f32(f32_to_bf16(x));
    fv<N> o;
#pragma unroll
    for (int j = 0; j < N; ++j) o.v[j] = r;
    return o;
  }
  __device__ __forceinline__ static fv<N> load(const bf16_t* p) {
    const raw x = *reinterpret_cast<const raw*>(p);
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&x);
    fv<N> o;
#pragma unroll
    for (int q = 0; q < N / 2; ++q) {
      o.v[2 * q] = __uint_as_float(w[q] << 16);
      o.v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
    }
    return o;
  }
  __device__ __forceinline__ static void store(bf16_t* p, const fv<N>& a) {
    raw x;
    uint32_t* w = reinterpret_cast<uint32_t*>(&x);
#pragma unroll
    for (int q = 0; q < N / 2; ++q) w[q] = pack_bf16x2(a.v[2 * q], a.v[2 * q + 1]);
    *reinterpret_cast<raw*>(p) = x;
  }
  __device__ __forceinline__ static void store_nt(bf16_t* p, const fv<N>& a) {
#pragma unroll
    for (int q = 0; q < N / 2; ++q)
      __builtin_nontemporal_store(pack_bf16x2(a.v[2 * q], a.v[2 * q + 1]), reinterpret_cast<uint32_t*>(p) + q);
  }
  // Gradient stores: stochastic rounding (pack_bf16x2_sr); idx = index of element 0.
  __device__ __forceinline__ static void store_grad(bf16_t* p, const fv<N>& a, uint32_t idx, uint32_t salt) {
    raw x;
    uint32_t* w = reinterpret_cast<uint32_t*>(&x);
#pragma unroll
    for (int q = 0; q < N / 2; ++q) w[q] = pack_bf16x2_sr(a.v[2 * q], a.v[2 * q + 1], idx + 2 * q, salt);
    *reinterpret_cast<raw*>(p) = x;
  }
  __device__ __forceinline__ static void store_grad_nt(bf16_t* p, const fv<N>& a, uint32_t idx, uint32_t salt) {
#pragma unroll
    for (int q = 0; q < N / 2; ++q)
      __builtin_nontemporal_store(pack_bf16x2_sr(a.v[2 * q], a.v[2 * q + 1], idx + 2 * q, salt),
                                  reinterpret_cast<uint32_t*>(p) + q);
  }
  // Two gradients of the same elements, rounded with one hash per element pair
  // (pack2_bf16x2_sr); idx = index of element 0 plus the call site's salt.
  __device__ __forceinline__ static void store_grad2_nt(bf16_t* pa, const fv<N>& a, bf16_t* pb, const fv<N>& b,
                                                        uint32_t idx) {
#pragma unroll
    for (int q = 0; q < N / 2; ++q) {
      uint32_t wa, wb;
      pack2_bf16x2_sr(a.v[2 * q], a.v[2 * q + 1], b.v[2 * q], b.v[2 * q + 1], idx + 2 * q, wa, wb);
      __builtin_nontemporal_store(wa, reinterpret_cast<uint32_t*>(pa) + q);
      __builtin_nontemporal_store(wb, reinterpret_cast<uint32_t*>(pb) + q);
    }
  }
};

template <typename T> using io4 = iov<T, 4>;

// ---------------------------------------------------------------- gate math
//
// minGRU gate math in linear space (reference mingru/minGRU.py:24-28, :56-60):
//   z = sigmoid(gate)  = exp(log_z),       log_z = -softplus(-gate)
//   a = 1 - z          = exp(log_coeffs),  log_coeffs = -softplus(gate)
//   g(x) = x + 0.5 (x >= 0), sigmoid(x) (x < 0)   = exp(log_g(x))
//   v = z g(hidden)    = exp(log_values)
// With e = exp(-gate), e2 = exp(-|hidden|), P = 1 + e, Q = 1 + e2 and
// R = 1 / (P Q) (one reciprocal for both sigmoids; Q cancels in z):
//   z = R Q,  a = e z,  v = (hidden + 0.5) z  (hidden >= 0)  |  e2 R  (hidden < 0).
// e is clamped at 2^100 (gate < -69.3), so P Q and R stay normal numbers:
// there z = 2^-100 instead of e^gate, and a rounds to 1. Rows past the end
// of the sequence are loaded as gate = -inf, hidden = 0, which gives
// a = 1 and v < 2^-100: the identity step up to that residue.

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaxExp2 = 100.0f;

__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

struct GateTerms {
  float e, e2, P, Q, R;
};

__device__ __forceinline__ GateTerms gate_terms(float gate, float hid) {
  GateTerms t;
  t.e = exp2_raw(fminf(gate * -kLog2e, kMaxExp2));
  t.e2 = exp2_raw(fabsf(hid) * -kLog2e);  // e^-|hidden|; only used when hidden < 0
  t.P = 1.0f + t.e;
  t.Q = 1.0f + t.e2;
  t.R = __builtin_amdgcn_rcpf(t.P * t.Q);
  return t;
}

// Forward coefficients: h_t = a h_{t-1} + v.
__device__ __forceinline__ void fwd_coeffs(float gate, float hid, float& a, float& v) {
  const GateTerms t = gate_terms(gate, hid);
  const float z = t.R * t.Q;
  a = t.e * z;
  v = hid >= 0.0f ? (hid + 0.5f) * z : t.e2 * t.R;
}

// Backward adds z and q = z g'(hidden), with g' as autograd of the
// reference's log_g sees it: 1 for x > 0, 0 at x == 0 (relu'(0) = 0),
// sigmoid(x) (1 - sigmoid(x)) for x < 0.
__device__ __forceinline__ void bwd_coeffs(float gate, float hid, float& a, float& z, float& v, float& q) {
  const GateTerms t = gate_terms(gate, hid);
  z = t.R * t.Q;
  a = t.e * z;
  const float vneg = t.e2 * t.R;             // z sigmoid(x)
  v = hid >= 0.0f ? (hid + 0.5f) * z : vneg;
  const float qneg = vneg * (t.R * t.P);     // z sigmoid(x) (1 - sigmoid(x))
  q = hid > 0.0f ? z : (hid < 0.0f ? qneg : 0.0f);
}

// ---------------------------------------------------------------- GELU

// erf(u) for u >= 0 by Abramowitz & Stegun, Handbook of Mathematical
// Functions (1964), formula 7.1.26: 1 - t (a1 + t (a2 + ... + t a5)) e^{-u^2},
// t = 1 / (1 + p u), absolute error <= 1.5e-7 -- far below the bf16 rounding
// these epilogues end in. Branch-free, one exp and one reciprocal; e^{-u^2}
// is returned too (GELU's derivative needs it).
__device__ __forceinline__ float erf_pos(float u, float& eu2) {
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * u);
  const float poly = t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  eu2 = exp2_raw(-u * u * kLog2e);
  return 1.0f - poly * eu2;
}

// gelu(x) = x/2 (1 + erf(x / sqrt 2)), the exact form of nn.GELU(), evaluated in
// fp32 in the order torch evaluates it (x * 0.5 * (1 + erf(x * 1/sqrt 2))),
// with the device library's erff. Every forward GELU of this library calls it
// (or reads the table gemm.hip fills from it), so all paths give the same bits.
__device__ __forceinline__ float gelu(float x) { return x * 0.5f * (1.0f + erff(x * 0.70710678118654752f)); }

// gelu'(x) = (1 + erf(x / sqrt 2))/2 + x phi(x)
__device__ __forceinline__ float gelu_grad(float x) {
  float eu2;  // e^{-x^2/2}
  const float e = erf_pos(fabsf(x) * 0.70710678118654752f, eu2);
  return 0.5f * (1.0f + copysignf(e, x)) + x * 0.39894228040143268f * eu2;
}

// Partial column sums -> column sums: out[c] = sum_p part[p * C + c]
// (colsum.hip). Fixed summation order, so results are reproducible.
int launch_reduce_partials(const float* part, int P, int C, float* out, hipStream_t st);

// ---------------------------------------------------------------- look-back words
//
// One 64-bit word per (time tile, channel) carries a tile's scan state
// between workgroups: value (fp32 bits) in the high half, tag in the low
// half. An inclusive prefix has tag kTagIncl and its value is the carry
// itself; an aggregate (A, V) carries A's bits with the sign bit set (A is a
// product of a_t in [0, 1], so its sign bit and bit 30 are free). Bit 30 of
// either tag is the call parity: a workspace alternates parity from call to
// call, so words left by the previous call (or the zeros of a fresh
// workspace) read as "not ready" and the words need no clearing between
// calls.
constexpr uint32_t kTagIncl = 1u;
constexpr uint32_t kTagAggBit = 0x80000000u;
constexpr uint32_t kTagParity = 0x40000000u;

__device__ __forceinline__ void publish_agg(uint64_t* w, float A, float V, uint32_t parity) {
  uint64_t x = (static_cast<uint64_t>(__float_as_uint(V)) << 32) |
               static_cast<uint64_t>(__float_as_uint(A) | kTagAggBit | (parity ? kTagParity : 0u));
  __hip_atomic_store(w, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void publish_incl(uint64_t* w, float V, uint32_t parity) {
  uint64_t x = (static_cast<uint64_t>(__float_as_uint(V)) << 32) |
               static_cast<uint64_t>(kTagIncl | (parity ? kTagParity : 0u));
  __hip_atomic_store(w, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t poll_word(const uint64_t* w) {
  return __hip_atomic_load(const_cast<uint64_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mg
