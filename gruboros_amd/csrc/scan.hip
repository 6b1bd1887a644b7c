// minGRU gate math + associative scan, forward and backward, for gfx950.
//
// Reference: mingru/minGRU.py:16-20 (heinsen_associative_scan_log),
// :24-28 (g, log_g), :47-69 (minGRU.forward). The reference evaluates
//   h = exp(a* + logcumsumexp(log_values - a*)),  a* = cumsum(log_coeffs)
// in log space. Here the same recurrence h_t = a_t h_{t-1} + z_t g(hidden_t)
// is evaluated in linear space with fp32 state: every term is a convex
// combination of positive numbers, so the linear form carries no
// cancellation (the log-space form loses ~|a*| * 2^-24 relative accuracy).
//
// Work decomposition (one pass over HBM per direction):
//   * A tile is a run of consecutive time steps x 64 consecutive channels of
//     one batch row; one workgroup per tile. Thread (cl, s) owns 4 adjacent
//     channels (one 8-byte bf16 / 16-byte fp32 vector per row) and a run of
//     consecutive time steps; 16 lanes cover 64 channels, so every row
//     segment a wave touches is a full 128-byte line for bf16.
//   * Each thread scans its run in registers, giving the run's affine map
//     h -> A h + V. The runs of a tile are combined by a Hillis-Steele scan
//     in LDS; the tile's map goes to later tiles through look-back words in
//     the workspace (decoupled look-back). Each chain of tiles (one channel
//     block) takes tickets from its own atomic counter, so a tile only ever
//     waits on tiles of its chain that were started before it.
//   * The workspace is zeroed once (mg_scan_workspace_init) and then kept
//     consistent by the kernels: the tile that draws a chain's last ticket
//     resets the count and flips the chain's parity bit (bit 31 of the
//     counter), and look-back words carry the parity of the call that wrote
//     them. Every word a call reads was written by the previous call of the
//     same direction (or is zero), so stale words never look ready and no
//     clearing kernel runs per call.
//   * The workspace starts with a header (magic, shape, error word, wait
//     limit) written by the initialisation. Every workgroup checks the
//     header against its launch and returns at once on a mismatch; every
//     look-back wait gives up after the header's poll limit. Either event
//     sets a bit in the header's error word (read by
//     mg_scan_workspace_check), so a workspace that was never initialised,
//     was initialised for another shape, or is shared by overlapping calls
//     ends the kernel with an error instead of a wait that never ends.
//   * The backward walks tiles in reverse time order with the adjoint
//     recurrence. It needs h_{t-1}: it reads the state entering each 8-step
//     pair of runs once (the forward's fp32 checkpoint when the output is
//     bf16, else the fp32 output itself) and rebuilds the states in fp32
//     from it; the first run of a pair hands its final state to the second.
//     (A bf16-rounded state would not do: at small gates dgate depends on
//     g(hidden) - h_{t-1}, a difference of two nearly equal numbers.)

#include <algorithm>
#include <mutex>

#include "mg_common.h"

namespace mg {
namespace scan {

constexpr int kVec = 4;                   // channels per thread
constexpr int kChLanes = 16;              // threads across channels
constexpr int kTileCh = kChLanes * kVec;  // 64 channels per tile

// Forward tiles: 16 runs of 8 steps (256 threads, 128 steps). The backward
// keeps three values per element plus the incoming gradient, so it uses
// shorter runs: 16 runs of 4 steps (256 threads, 64 steps).
#ifndef MG_SCAN_BWD_SUBS
#define MG_SCAN_BWD_SUBS 16
#define MG_SCAN_BWD_ROWS 4
#endif
#ifndef MG_SCAN_FWD_SUBS
#define MG_SCAN_FWD_SUBS 16
#endif
constexpr int kFwdSubs = MG_SCAN_FWD_SUBS, kFwdRows = 8;
constexpr int kBwdSubs = MG_SCAN_BWD_SUBS, kBwdRows = MG_SCAN_BWD_ROWS;
constexpr int kFwdTileRows = kFwdSubs * kFwdRows;
// fp32 state checkpoints (optional forward output, backward input): the state
// after every kCkptRows-th step, i.e. the state entering every second
// backward run; the run in between gets its entering state from its
// neighbour through LDS.
constexpr int kCkptRows = 8;
static_assert(2 * kBwdRows == kCkptRows && kFwdRows % kCkptRows == 0, "checkpoint spacing");
constexpr int kBwdTileRows = kBwdSubs * kBwdRows;

struct Geometry {
  int B, T, Di;
  int nblk_d;    // channel blocks per batch row
  int ncb;       // chains = channel blocks in total (B * nblk_d)
  int tile_rows; // time steps per tile (direction dependent)
  int ntiles;    // time tiles per chain
  int64_t BD;    // B * Di
};

// Workspace: a 256-byte header, ticket counters (one per chain and
// direction), then one look-back word per (tile, channel) for the forward
// tiles, then the same for the backward tiles.
constexpr uint32_t kWsMagic = 0x4d475343u;  // "MGSC"
constexpr uint32_t kErrShape = 1u;          // header missing or for another shape
constexpr uint32_t kErrTicket = 2u;         // a ticket past the chain's last tile
constexpr uint32_t kErrStall = 4u;          // a look-back wait gave up
constexpr uint32_t kDefaultPolls = 1u << 22;  // ~1-4 s of polling

struct WsHeader {
  uint32_t magic;
  int32_t B, T, Di;
  uint32_t err;          // kErr* bits, set by the kernels (atomic or)
  uint32_t max_polls;    // look-back polls of one word before giving up
  uint32_t pad[58];
};
static_assert(sizeof(WsHeader) == 256, "header size");

inline size_t ws_header_bytes(int ncb) {
  return sizeof(WsHeader) + (static_cast<size_t>(ncb) * 2 * 4 + 255) / 256 * 256;
}

// The header matches this launch; otherwise the error bit is set (by one
// thread) and the caller returns. Wave-uniform.
__device__ __forceinline__ bool header_ok(WsHeader* h, const Geometry& g) {
  const bool ok = h->magic == kWsMagic && h->B == g.B && h->T == g.T && h->Di == g.Di;
  if (!ok && threadIdx.x == 0) atomicOr(&h->err, kErrShape);
  return ok;
}

// Chain and tile of this workgroup. The chain comes from the block index; the
// tile (time position) from the chain's ticket counter, in start order. The
// results are wave-uniform, so tile base addresses live in scalar registers.
// The counter's bit 31 is the chain's parity for this call; the draw of the
// last ticket resets the count and flips the parity for the next call (no
// other draw of this call follows it, and the next call starts after this
// kernel has finished).
constexpr uint32_t kParityBit = 0x80000000u;
// Returns false (after setting the error bit) for a ticket past the chain's
// last tile, which only a corrupted counter gives; the workgroup then exits.
__device__ __forceinline__ bool take_tile(const Geometry& g, WsHeader* hdr, uint32_t* counters, uint32_t* s_ticket,
                                          bool reverse, int& k, int& b, int& d0, uint32_t& parity) {
  const int cbi = static_cast<int>(blockIdx.x % static_cast<uint32_t>(g.ncb));
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(counters + cbi, 1u);
    if ((old & ~kParityBit) == static_cast<uint32_t>(g.ntiles - 1)) atomicExch(counters + cbi, (old & kParityBit) ^ kParityBit);
    *s_ticket = old;
  }
  __syncthreads();
  const uint32_t t = __builtin_amdgcn_readfirstlane(*s_ticket);
  parity = t >> 31;
  const int kk = static_cast<int>(t & ~kParityBit);
  if (kk >= g.ntiles) {
    if (threadIdx.x == 0) atomicOr(&hdr->err, kErrTicket);
    return false;
  }
  k = reverse ? (g.ntiles - 1 - kk) : kk;
  b = cbi / g.nblk_d;
  d0 = (cbi % g.nblk_d) * kTileCh;
  return true;
}

// The state entering tile k of channel c (one channel per lane), from the
// look-back words of the tiles before it in scan order (step -1: earlier
// tiles, forward scan; +1: later tiles, backward scan). `last` is the chain's
// end tile in that direction (0 or ntiles - 1); it only ever publishes an
// inclusive prefix, and the walk never steps past it.
//   1. Walk back until an inclusive prefix I_j is found (aggregates on the
//      way are passed over).
//   2. Compose forward from it: c = A_i c + V_i for each tile i between j and
//      k, re-reading each word. A word that has meanwhile become inclusive
//      holds exactly that value (tile i computed it as A_i c + V_i from the
//      same c), so the carry is the one a strictly sequential chain computes,
//      bit for bit, whatever the timing (folding the aggregates during the
//      walk would round (A_1 A_2) I instead of A_1 (A_2 I)).
// A word that stays not-ready for max_polls polls ends the wait: the error
// bit is set and 0 is returned (the results are then wrong, and the caller
// learns it from mg_scan_workspace_check).
__device__ __forceinline__ float look_back1(const uint64_t* status, int64_t BD, int64_t c, int k, int step, int last,
                                            uint32_t parity, uint32_t max_polls, uint32_t* err) {
  const uint64_t* base = status + c;
  const uint32_t par = parity ? kTagParity : 0u;
  int j = k + step;
  uint32_t polls = 0;
  float carry;
  while (true) {
    const uint64_t x = poll_word(base + static_cast<int64_t>(j) * BD);
    const uint32_t tag = static_cast<uint32_t>(x);
    if (tag == (kTagIncl | par)) {
      carry = __uint_as_float(static_cast<uint32_t>(x >> 32));
      break;
    }
    if (j != last && (tag & (kTagAggBit | kTagParity)) == (kTagAggBit | par)) {
      j += step;
      polls = 0;
    } else {
      if (++polls > max_polls) {
        atomicOr(err, kErrStall);
        return 0.0f;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  for (int i = j - step; i != k; i -= step) {  // every word here was seen ready (an aggregate)
    const uint64_t x = poll_word(base + static_cast<int64_t>(i) * BD);
    const uint32_t tag = static_cast<uint32_t>(x);
    const float v = __uint_as_float(static_cast<uint32_t>(x >> 32));
    carry = tag == (kTagIncl | par) ? v : __builtin_fmaf(__uint_as_float(tag & ~(kTagAggBit | kTagParity)), carry, v);
  }
  return carry;
}

// Load one run of rows. hb/gb are tile base pointers (wave-uniform), off is
// this thread's first element relative to them, ld the row stride; all
// offsets inside a tile fit in 32 bits. Rows at or past T (and channels past
// Di) read as gate = -inf, hidden = 0, which the gate math turns into the
// identity step. Full runs (all but the tail of the sequence) load unmasked.
// A 4-channel load that bypasses the caches' retention (non-temporal), for
// inputs far larger than the caches (bf16; fp32 loads stay plain).
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
template <typename Tin>
__device__ __forceinline__ f4 load4_nt(const Tin* p) {
  if constexpr (sizeof(Tin) == 2) {
    const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    f4 o;
    o.v[0] = __uint_as_float(x[0] << 16);
    o.v[1] = __uint_as_float(x[0] & 0xffff0000u);
    o.v[2] = __uint_as_float(x[1] << 16);
    o.v[3] = __uint_as_float(x[1] & 0xffff0000u);
    return o;
  } else {
    return io4<Tin>::load(p);
  }
}

// kNT: the full runs' loads are non-temporal.
template <typename Tin, int kRows, bool kNT = false>
__device__ __forceinline__ void load_run(const Tin* hb, const Tin* gb, int off, int ld, bool ok, int nrows,
                                         f4 (&hv)[kRows], f4 (&gv)[kRows]) {
  if (ok && nrows >= kRows) {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      if constexpr (kNT) {
        hv[i] = load4_nt<Tin>(hb + (off + i * ld));
        gv[i] = load4_nt<Tin>(gb + (off + i * ld));
      } else {
        hv[i] = io4<Tin>::load(hb + (off + i * ld));
        gv[i] = io4<Tin>::load(gb + (off + i * ld));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const bool live = ok && i < nrows;
      hv[i] = live ? io4<Tin>::load(hb + (off + i * ld)) : io4<Tin>::fill(0.0f);
      gv[i] = live ? io4<Tin>::load(gb + (off + i * ld)) : io4<Tin>::fill(-INFINITY);
    }
  }
}

template <typename Tg, int kRows>
__device__ __forceinline__ void load_grad(const Tg* pb, int off, int ld, bool ok, int nrows, f4 (&dv)[kRows]) {
  if (ok && nrows >= kRows) {
#pragma unroll
    for (int i = 0; i < kRows; ++i) dv[i] = io4<Tg>::load(pb + (off + i * ld));
  } else {
#pragma unroll
    for (int i = 0; i < kRows; ++i)
      dv[i] = (ok && i < nrows) ? io4<Tg>::load(pb + (off + i * ld)) : io4<Tg>::fill(0.0f);
  }
}

// Run maps of one tile in LDS, double-buffered for the scan across runs.
template <int kSubs>
struct RunMaps {
  f4 A[2][kSubs][kChLanes];
  f4 V[2][kSubs][kChLanes];
};

// Inclusive scan of the affine run maps (h -> A h + V) across the kSubs runs
// of a tile, Hillis-Steele over LDS with one barrier per doubling step. The
// forward scan composes earlier runs first; the reverse scan (backward pass)
// composes later runs first. Both use (A, V) <- (A A', A V' + V) with the
// partner's map (A', V'). Returns the buffer holding the inclusive maps.
template <int kSubs, bool kReverse>
__device__ __forceinline__ int scan_runs(RunMaps<kSubs>& m, int s, int cl, f4 A, f4 V) {
  int buf = 0;
  m.A[0][s][cl] = A;
  m.V[0][s][cl] = V;
  __syncthreads();
#pragma unroll
  for (int o = 1; o < kSubs; o <<= 1) {
    const int src = kReverse ? s + o : s - o;
    if (kReverse ? src < kSubs : src >= 0) {
      const f4 pa = m.A[buf][src][cl], pv = m.V[buf][src][cl];
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        V.v[j] = A.v[j] * pv.v[j] + V.v[j];
        A.v[j] = A.v[j] * pa.v[j];
      }
    }
    buf ^= 1;
    m.A[buf][s][cl] = A;
    m.V[buf][s][cl] = V;
    __syncthreads();
  }
  return buf;
}

// ------------------------------------------------------------------ forward

// kRes: the output is res + h (fp32, res with the output's strides): the scan
// state joins the residual stream here, and h itself is kept only as the fp32
// checkpoints the backward rebuilds it from.
template <typename Tin, typename Tout, bool kNT, bool kRes = false>
__global__ __launch_bounds__(kChLanes * kFwdSubs) void scan_fwd_kernel(
    const Tin* __restrict__ hidden, const Tin* __restrict__ gate, int64_t in_sb, int64_t in_ld,
    const float* __restrict__ h0, Tout* __restrict__ hout, int64_t out_sb, int64_t out_ld,
    float* __restrict__ h_last, float* __restrict__ ckpt, Geometry g, WsHeader* __restrict__ hdr,
    uint32_t* __restrict__ counters, uint64_t* __restrict__ status, const float* __restrict__ res) {
  static_assert(!kRes || sizeof(Tout) == 4, "the residual sum is fp32");
  constexpr int kSubs = kFwdSubs, kRows = kFwdRows;
  __shared__ uint32_t s_ticket;
  __shared__ RunMaps<kSubs> s_maps;
  __shared__ f4 s_carry[kChLanes];

  const int tid = threadIdx.x;
  const int cl = tid % kChLanes;
  const int s = tid / kChLanes;
  int k, b, d0;
  uint32_t parity;
  if (!header_ok(hdr, g)) return;
  const uint32_t max_polls = hdr->max_polls;
  if (!take_tile(g, hdr, counters, &s_ticket, false, k, b, d0, parity)) return;
  const int d = d0 + cl * kVec;
  const bool ok = d < g.Di;
  const int t0 = k * kFwdTileRows + s * kRows;
  const int64_t c = static_cast<int64_t>(b) * g.Di + d;
  const int ild = static_cast<int>(in_ld), old = static_cast<int>(out_ld);
  const int64_t in_tile = b * in_sb + static_cast<int64_t>(k) * kFwdTileRows * in_ld + d0;

  f4 hv[kRows], gv[kRows];
  load_run<Tin, kRows, kNT>(hidden + in_tile, gate + in_tile, s * kRows * ild + cl * kVec, ild, ok, g.T - t0, hv, gv);

  float a[kRows][kVec], v[kRows][kVec];
  f4 A, V;
#pragma unroll
  for (int j = 0; j < kVec; ++j) { A.v[j] = 1.0f; V.v[j] = 0.0f; }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      fwd_coeffs(gv[i].v[j], hv[i].v[j], a[i][j], v[i][j]);
      V.v[j] = a[i][j] * V.v[j] + v[i][j];
      A.v[j] = A.v[j] * a[i][j];
    }
  }
  // kRes: the run's residual rows in two batches of half a run (all at once
  // would cost a wave per SIMD); the first is requested before the look-back,
  // so that it lands under it
  constexpr int kHalf = kRows / 2;
  const int64_t out_off =
      (b * out_sb + static_cast<int64_t>(k) * kFwdTileRows * out_ld + d0) + (s * kRows * static_cast<int>(out_ld) + cl * kVec);
  f4 rv[kRes ? kHalf : 1];
  auto load_res = [&](int i0) {
    if constexpr (kRes) {
#pragma unroll
      for (int i = 0; i < kHalf; ++i)
        rv[i] = (ok && t0 + i0 + i < g.T) ? io4<float>::load(res + out_off + (i0 + i) * static_cast<int>(out_ld))
                                           : io4<float>::fill(0.0f);
    }
  };
  const int buf = scan_runs<kSubs, false>(s_maps, s, cl, A, V);
  load_res(0);

  // Wave 0 links the tile into its chain, one channel per lane: lane
  // (s, cl) takes channel cl * 4 + s.
  if (tid < 64 && ok) {
    const float TA = reinterpret_cast<const float*>(&s_maps.A[buf][kSubs - 1][cl])[s];
    const float TV = reinterpret_cast<const float*>(&s_maps.V[buf][kSubs - 1][cl])[s];
    uint64_t* st = status + static_cast<int64_t>(k) * g.BD + c + s;
    float carry;
    if (k == 0) {
      carry = h0 ? h0[c + s] : 0.0f;
    } else {
      publish_agg(st, TA, TV, parity);
      carry = look_back1(status, g.BD, c + s, k, -1, 0, parity, max_polls, &hdr->err);
    }
    if (k + 1 < g.ntiles) publish_incl(st, __builtin_fmaf(TA, carry, TV), parity);  // as look_back1 composes
    reinterpret_cast<float*>(&s_carry[cl])[s] = carry;
  }
  __syncthreads();
  if (!ok) return;

  f4 h = s_carry[cl];
  if (s > 0) {
    const f4 pa = s_maps.A[buf][s - 1][cl], pv = s_maps.V[buf][s - 1][cl];
#pragma unroll
    for (int j = 0; j < kVec; ++j) h.v[j] = pa.v[j] * h.v[j] + pv.v[j];
  }
  Tout* ob = hout + out_off;
  // kFull: every row of the run is inside the sequence (all runs but the
  // tail's), so the stores need no per-row test.
  auto outputs = [&](auto full_tag) {
    constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      if (kRes && i == kHalf) {
        __builtin_amdgcn_sched_barrier(0);
        load_res(kHalf);
      }
#pragma unroll
      for (int j = 0; j < kVec; ++j) h.v[j] = a[i][j] * h.v[j] + v[i][j];
      if constexpr (kRes) {
        f4 o;
#pragma unroll
        for (int j = 0; j < kVec; ++j) o.v[j] = rv[i % kHalf].v[j] + h.v[j];
        if (kFull || t0 + i < g.T) io4<Tout>::store_nt(ob + i * old, o);
      } else {
        if (kFull || t0 + i < g.T) io4<Tout>::store_nt(ob + i * old, h);
      }
      if (!kFull && h_last && t0 + i == g.T - 1) io4<float>::store(h_last + c, h);
      if (ckpt && (i + 1) % kCkptRows == 0 && (kFull || t0 + i < g.T))
        io4<float>::store(ckpt + static_cast<int64_t>((t0 + i) / kCkptRows) * g.BD + c, h);
    }
    if (kFull && h_last && t0 + kRows == g.T) io4<float>::store(h_last + c, h);
  };
  if (t0 + kRows <= g.T)
    outputs(std::true_type{});
  else
    outputs(std::false_type{});
}

// ------------------------------------------------------------------ backward

// Four channels of one row kept as loaded (bf16 stays packed, two per
// register) until each value is needed, to keep the backward's register
// footprint small enough for six waves per SIMD.
template <typename T> struct Raw4;
template <> struct Raw4<bf16_t> {
  uint2 r;
  __device__ __forceinline__ static Raw4 load(const bf16_t* p) { return Raw4{*reinterpret_cast<const uint2*>(p)}; }
  __device__ __forceinline__ static Raw4 fill(float f) {
    const uint32_t b = f32_to_bf16(f);
    return Raw4{make_uint2(b | (b << 16), b | (b << 16))};
  }
  __device__ __forceinline__ float get(int j) const {
    const uint32_t w = j < 2 ? r.x : r.y;
    return (j & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
  }
};
template <> struct Raw4<float> {
  float4 r;
  __device__ __forceinline__ static Raw4 load(const float* p) { return Raw4{*reinterpret_cast<const float4*>(p)}; }
  __device__ __forceinline__ static Raw4 fill(float f) { return Raw4{make_float4(f, f, f, f)}; }
  __device__ __forceinline__ float get(int j) const { return j == 0 ? r.x : j == 1 ? r.y : j == 2 ? r.z : r.w; }
};

template <typename T, int kRows>
__device__ __forceinline__ void load_raw(const T* base, int off, int ld, bool ok, int nrows, float pad,
                                         Raw4<T> (&v)[kRows]) {
  if (ok && nrows >= kRows) {
#pragma unroll
    for (int i = 0; i < kRows; ++i) v[i] = Raw4<T>::load(base + (off + i * ld));
  } else {
#pragma unroll
    for (int i = 0; i < kRows; ++i)
      v[i] = (ok && i < nrows) ? Raw4<T>::load(base + (off + i * ld)) : Raw4<T>::fill(pad);
  }
}

// Two passes over each thread's 4-step run, with the inputs held raw:
//   1. a_t and z_t from the gate (kept), the run's reverse map for mu_t =
//      a_t lambda_t, lambda_t = dh_t + mu_{t+1}; scan across runs and tiles.
//   2. lambda_t down the run, then up the run with h_{t-1} rebuilt in fp32
//      from the state entering the run: g~, g' from the hidden input,
//      dgate = lambda a z (g~ - h_{t-1}), dhidden = lambda z g'(hidden).
template <typename Tin, typename Th>
__global__ __launch_bounds__(kChLanes * kBwdSubs) void scan_bwd_kernel(
    const Tin* __restrict__ hidden, const Tin* __restrict__ gate, int64_t in_sb, int64_t in_ld,
    const float* __restrict__ h0, const Th* __restrict__ hout, int64_t out_sb, int64_t out_ld,
    const float* __restrict__ ckpt, const Th* __restrict__ dh, int64_t g_sb, int64_t g_ld,
    const float* __restrict__ dh_last,
    Tin* __restrict__ dhidden, Tin* __restrict__ dgate, int64_t d_sb, int64_t d_ld, float* __restrict__ dh0,
    Geometry g, WsHeader* __restrict__ hdr, uint32_t* __restrict__ counters, uint64_t* __restrict__ status) {
  constexpr int kSubs = kBwdSubs, kRows = kBwdRows;
  __shared__ uint32_t s_ticket;
  __shared__ RunMaps<kSubs> s_maps;
  __shared__ f4 s_carry[kChLanes];
  __shared__ f4 s_hmid[kSubs / 2][kChLanes];

  // Runs 0, 2, 4, ... (each the first of a checkpoint interval) sit in the
  // first half of the workgroup and 1, 3, 5, ... in the second, so the extra
  // work of the first runs fills whole waves.
  const int tid = threadIdx.x;
  const int cl = tid % kChLanes;
  const int s = ((tid / kChLanes) % (kSubs / 2)) * 2 + tid / (kChLanes * kSubs / 2);
  int k, b, d0;
  uint32_t parity;
  if (!header_ok(hdr, g)) return;
  const uint32_t max_polls = hdr->max_polls;
  if (!take_tile(g, hdr, counters, &s_ticket, true, k, b, d0, parity)) return;
  const int d = d0 + cl * kVec;
  const bool ok = d < g.Di;
  const int t0 = k * kBwdTileRows + s * kRows;
  const int64_t c = static_cast<int64_t>(b) * g.Di + d;
  const int ild = static_cast<int>(in_ld), gld = static_cast<int>(g_ld);
  const int64_t in_tile = b * in_sb + static_cast<int64_t>(k) * kBwdTileRows * in_ld + d0;
  const int in_off = s * kRows * ild + cl * kVec;

  Raw4<Tin> hr[kRows], gr[kRows];
  Raw4<Th> dr[kRows];
  load_raw<Tin, kRows>(gate + in_tile, in_off, ild, ok, g.T - t0, -INFINITY, gr);
  load_raw<Tin, kRows>(hidden + in_tile, in_off, ild, ok, g.T - t0, 0.0f, hr);
  load_raw<Th, kRows>(dh + (b * g_sb + static_cast<int64_t>(k) * kBwdTileRows * g_ld + d0), s * kRows * gld + cl * kVec,
                      gld, ok, g.T - t0, 0.0f, dr);
  // h_{t0-1}: from the fp32 checkpoint for runs starting a checkpoint
  // interval (the other runs get it from their neighbour below), else the
  // forward output of the row before the run (exact for fp32 outputs); h0
  // (or 0) at t = 0.
  const bool from_left = ckpt && (s & 1);
  f4 hc = io4<float>::fill(0.0f);
  if (ok && t0 < g.T && !from_left) {
    if (t0 > 0)
      hc = ckpt ? io4<float>::load(ckpt + static_cast<int64_t>(t0 / kCkptRows - 1) * g.BD + c)
                : io4<Th>::load(hout + (b * out_sb + static_cast<int64_t>(t0 - 1) * out_ld + d));
    else if (h0)
      hc = io4<float>::load(h0 + c);
  }
  float a[kRows][kVec], z[kRows][kVec];
  f4 A, M;
#pragma unroll
  for (int j = 0; j < kVec; ++j) { A.v[j] = 1.0f; M.v[j] = 0.0f; }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const float e = exp2_raw(fminf(gr[i].get(j) * -kLog2e, kMaxExp2));
      z[i][j] = __builtin_amdgcn_rcpf(1.0f + e);
      a[i][j] = e * z[i][j];
    }
  }
  // The first run of a checkpoint interval passes its final state on.
  if (ckpt && !(s & 1)) {
    f4 he = hc;
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const float x = hr[i].get(j);
        const float e2 = exp2_raw(fabsf(x) * -kLog2e);
        const float gt = x >= 0.0f ? x + 0.5f : e2 * __builtin_amdgcn_rcpf(1.0f + e2);
        he.v[j] = a[i][j] * he.v[j] + z[i][j] * gt;
      }
    }
    s_hmid[s / 2][cl] = he;
  }
  // Reverse run map mu -> A mu + M.
#pragma unroll
  for (int i = kRows - 1; i >= 0; --i) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      M.v[j] = a[i][j] * (dr[i].get(j) + M.v[j]);
      A.v[j] = A.v[j] * a[i][j];
    }
  }
  const int buf = scan_runs<kSubs, true>(s_maps, s, cl, A, M);

  // Wave 0 links the tile into its chain, one channel per lane: lane
  // (q, cl) takes channel cl * 4 + q.
  if (tid < 64 && ok) {
    const int q = tid / kChLanes;
    const float TA = reinterpret_cast<const float*>(&s_maps.A[buf][0][cl])[q];
    const float TM = reinterpret_cast<const float*>(&s_maps.V[buf][0][cl])[q];
    uint64_t* st = status + static_cast<int64_t>(k) * g.BD + c + q;
    // The gradient arriving at h_last enters as the carry into the chain's
    // last tile: every row past T - 1 is an identity step (a = 1, dh = 0), so
    // it reaches row T - 1 unchanged and joins dh there, as it should.
    float carry = 0.0f;
    if (k == g.ntiles - 1) {
      if (dh_last) carry = dh_last[c + q];
    } else {
      publish_agg(st, TA, TM, parity);
      carry = look_back1(status, g.BD, c + q, k, +1, g.ntiles - 1, parity, max_polls, &hdr->err);
    }
    if (k > 0) publish_incl(st, __builtin_fmaf(TA, carry, TM), parity);  // as look_back1 composes
    reinterpret_cast<float*>(&s_carry[cl])[q] = carry;
  }
  __syncthreads();
  if (!ok) return;

  f4 mu = s_carry[cl];
  if (s + 1 < kSubs) {
    const f4 pa = s_maps.A[buf][s + 1][cl], pm = s_maps.V[buf][s + 1][cl];
#pragma unroll
    for (int j = 0; j < kVec; ++j) mu.v[j] = pa.v[j] * mu.v[j] + pm.v[j];
  }
  if (from_left) hc = s_hmid[s / 2][cl];
  float lam[kRows][kVec];
#pragma unroll
  for (int i = kRows - 1; i >= 0; --i) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      lam[i][j] = dr[i].get(j) + mu.v[j];
      mu.v[j] = a[i][j] * lam[i][j];
    }
  }
  if (dh0 && t0 == 0) io4<float>::store(dh0 + c, mu);

  const int dld = static_cast<int>(d_ld);
  const int64_t d_tile = b * d_sb + static_cast<int64_t>(k) * kBwdTileRows * d_ld + d0;
  const int d_off = s * kRows * dld + cl * kVec;
  Tin* dhb = dhidden + d_tile + d_off;
  Tin* dgb = dgate + d_tile + d_off;
  // bf16 gradients round stochastically (mg_common.h), keyed by the element's
  // (b, t, d) index (mod 2^32) plus a salt for this call site
  const uint32_t idx0 = (static_cast<uint32_t>(b) * static_cast<uint32_t>(g.T) + static_cast<uint32_t>(t0)) *
                            static_cast<uint32_t>(g.Di) + static_cast<uint32_t>(d) + 0x5a17u;
  // kFull: every row of the run is inside the sequence (all runs but the
  // tail's), so the stores need no per-row test.
  auto outputs = [&](auto full_tag) {
    constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      f4 og, oh;
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        // g~ = g(hidden), gp = g'(hidden) (0 at hidden = 0, as autograd of relu gives)
        const float x = hr[i].get(j);
        const float e2 = exp2_raw(fabsf(x) * -kLog2e);
        const float r2 = __builtin_amdgcn_rcpf(1.0f + e2);
        const float sig = e2 * r2;  // sigmoid(x) for x < 0
        const float gt = x >= 0.0f ? x + 0.5f : sig;
        const float gp = x > 0.0f ? 1.0f : (x < 0.0f ? sig * r2 : 0.0f);
        const float vv = z[i][j] * gt;
        og.v[j] = lam[i][j] * (a[i][j] * (vv - z[i][j] * hc.v[j]));
        oh.v[j] = lam[i][j] * (z[i][j] * gp);
        hc.v[j] = a[i][j] * hc.v[j] + vv;
      }
      if (kFull || t0 + i < g.T)
        io4<Tin>::store_grad2_nt(dgb + i * dld, og, dhb + i * dld, oh, idx0 + static_cast<uint32_t>(i * g.Di));
    }
  };
  if (t0 + kRows <= g.T)
    outputs(std::true_type{});
  else
    outputs(std::false_type{});
}

// ------------------------------------------------------------------ host

// Workspace initialisation: zeros, then the header (one thread; the header
// block is skipped by the zero fill).
__global__ void init_kernel(uint4* __restrict__ p, int64_t n16, int B, int T, int Di, uint32_t max_polls) {
  constexpr int64_t kHdr16 = sizeof(WsHeader) / 16;
  for (int64_t i = kHdr16 + blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && threadIdx.x < kHdr16) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (threadIdx.x == 0) v = make_uint4(kWsMagic, static_cast<uint32_t>(B), static_cast<uint32_t>(T), static_cast<uint32_t>(Di));
    if (threadIdx.x == 1) v = make_uint4(0u, max_polls, 0u, 0u);
    p[threadIdx.x] = v;
  }
}

__global__ void set_polls_kernel(WsHeader* h, uint32_t max_polls) { h->max_polls = max_polls; }

inline void make_geometry(int B, int T, int Di, int tile_rows, Geometry& g) {
  g.B = B; g.T = T; g.Di = Di;
  g.nblk_d = (Di + kTileCh - 1) / kTileCh;
  g.ncb = B * g.nblk_d;
  g.tile_rows = tile_rows;
  g.ntiles = (T + tile_rows - 1) / tile_rows;
  g.BD = static_cast<int64_t>(B) * Di;
}

// One workspace serves both directions: counters for both, then the forward
// words, then the backward words.
inline size_t ws_bytes_any(int B, int T, int Di) {
  Geometry f, b;
  make_geometry(B, T, Di, kFwdTileRows, f);
  make_geometry(B, T, Di, kBwdTileRows, b);
  return ws_header_bytes(f.ncb) + static_cast<size_t>(f.ntiles + b.ntiles) * f.BD * sizeof(uint64_t);
}

// `need`: the workspace bytes the call requires (0: both directions' size)
inline int check_common(const char* fn, int B, int T, int Di, int tile_rows, void* ws, size_t ws_size,
                        Geometry& g, size_t need = 0) {
  if (B < 1 || T < 1 || Di < 4) return fail(MG_ERR_ARG, "%s: bad shape B=%d T=%d Di=%d", fn, B, T, Di);
  if (Di % kVec) return fail(MG_ERR_ARG, "%s: Di=%d must be a multiple of 4", fn, Di);
  make_geometry(B, T, Di, tile_rows, g);
  const int64_t nblocks = static_cast<int64_t>(g.ncb) * g.ntiles;
  if (nblocks > 0x7fffffff) return fail(MG_ERR_ARG, "%s: problem too large (%lld tiles)", fn, (long long)nblocks);
  if (!need) need = ws_bytes_any(B, T, Di);
  if (!ws || ws_size < need)
    return fail(MG_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", fn, ws_size, need);
  if (!aligned(ws, 16)) return fail(MG_ERR_ARG, "%s: workspace not 16-byte aligned", fn);
  return MG_OK;
}

inline int check_tensor(const char* fn, const char* name, const void* p, int dtype, int64_t sb, int64_t ld) {
  if (!p) return fail(MG_ERR_ARG, "%s: %s is NULL", fn, name);
  if (dtype != MG_F32 && dtype != MG_BF16) return fail(MG_ERR_DTYPE, "%s: %s dtype %d unsupported", fn, name, dtype);
  if (sb % kVec || ld % kVec || sb < 0 || ld < 0)
    return fail(MG_ERR_ARG, "%s: %s strides (%lld, %lld) must be non-negative multiples of 4", fn, name,
                (long long)sb, (long long)ld);
  // offsets inside one tile are 32-bit
  if (static_cast<int64_t>(std::max(kFwdTileRows, kBwdTileRows)) * ld + kTileCh > 0x7fffffffLL)
    return fail(MG_ERR_ARG, "%s: %s row stride %lld too large", fn, name, (long long)ld);
  if (!aligned(p, dtype == MG_F32 ? 16 : 8)) return fail(MG_ERR_ARG, "%s: %s misaligned", fn, name);
  return MG_OK;
}

inline int check_f32vec(const char* fn, const char* name, const void* p) {
  if (p && !aligned(p, 16)) return fail(MG_ERR_ARG, "%s: %s not 16-byte aligned", fn, name);
  return MG_OK;
}

// Forward or backward counters and look-back words of a workspace.
inline WsHeader* ws_header(void* ws) { return static_cast<WsHeader*>(ws); }
inline uint32_t* ws_counters(void* ws, const Geometry& g, bool bwd) {
  return reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + sizeof(WsHeader)) + (bwd ? g.ncb : 0);
}
inline uint64_t* ws_status(void* ws, const Geometry& g, bool bwd) {
  uint64_t* w = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + ws_header_bytes(g.ncb));
  if (bwd) w += static_cast<int64_t>((g.T + kFwdTileRows - 1) / kFwdTileRows) * g.BD;
  return w;
}

// Inputs (hidden + gate) beyond this many bytes are read non-temporally by the
// forward: they cannot stay in the 256 MB Infinity Cache anyway (cfg2: 1 GiB;
// measured 5% faster there), while smaller ones, such as a training layer's
// projection output arriving warm from its product, keep the cached loads.
constexpr int64_t kFwdNtBytes = int64_t(512) << 20;

template <typename Tin, typename Tout>
void launch_fwd(const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld, const float* h0, void* h,
                int64_t out_sb, int64_t out_ld, float* h_last, float* ckpt, const Geometry& g, void* ws,
                hipStream_t st, const float* res = nullptr) {
  const bool nt = 2 * int64_t(sizeof(Tin)) * g.B * g.T * g.Di > kFwdNtBytes;
  auto kern = nt ? scan_fwd_kernel<Tin, Tout, true> : scan_fwd_kernel<Tin, Tout, false>;
  if constexpr (sizeof(Tout) == 4) {
    if (res) kern = nt ? scan_fwd_kernel<Tin, Tout, true, true> : scan_fwd_kernel<Tin, Tout, false, true>;
  }
  hipLaunchKernelGGL(kern, dim3(g.ncb * g.ntiles), dim3(kChLanes * kFwdSubs), 0, st,
                     static_cast<const Tin*>(hidden), static_cast<const Tin*>(gate), in_sb, in_ld, h0,
                     static_cast<Tout*>(h), out_sb, out_ld, h_last, ckpt, g, ws_header(ws),
                     ws_counters(ws, g, false), ws_status(ws, g, false), res);
}

template <typename Tin, typename Th>
void launch_bwd(const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld, const float* h0,
                const void* h, int64_t out_sb, int64_t out_ld, const float* ckpt, const void* dh, int64_t g_sb,
                int64_t g_ld,
                const float* dh_last, void* dhidden, void* dgate, int64_t d_sb, int64_t d_ld, float* dh0,
                const Geometry& g, void* ws, hipStream_t st) {
  hipLaunchKernelGGL((scan_bwd_kernel<Tin, Th>), dim3(g.ncb * g.ntiles), dim3(kChLanes * kBwdSubs), 0, st,
                     static_cast<const Tin*>(hidden), static_cast<const Tin*>(gate), in_sb, in_ld, h0,
                     static_cast<const Th*>(h), out_sb, out_ld, ckpt, static_cast<const Th*>(dh), g_sb, g_ld, dh_last,
                     static_cast<Tin*>(dhidden), static_cast<Tin*>(dgate), d_sb, d_ld, dh0, g, ws_header(ws),
                     ws_counters(ws, g, true), ws_status(ws, g, true));
}

// ------------------------------------------------------------------ allocation-free forward
//
// mg_scan_fwd_noalloc keeps its look-back workspace in this file-scope device
// array instead of a caller's workspace. Each device holds its own copy (at
// its own address, found once per device with hipGetSymbolAddress); every
// call re-initialises the part it uses with the init kernel (a kernel, not a
// memset: callers may capture the call into a graph). Calls on one device
// share the array, so calls that may overlap on one device race.
constexpr size_t kNoAllocBytes = (size_t(16) << 20) + (size_t(64) << 10);  // 16 MiB + 64 KiB
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call per device).
inline int scratch_ptr(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MG_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MG_ERR_ARG, "%s: device %d beyond %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MG_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MG_OK;
}

// Bytes of a forward-only workspace (header, counters, forward look-back words).
inline size_t fwd_ws_bytes(int B, int T, int Di) {
  Geometry f;
  make_geometry(B, T, Di, kFwdTileRows, f);
  return ws_header_bytes(f.ncb) + static_cast<size_t>(f.ntiles) * f.BD * sizeof(uint64_t);
}

}  // namespace scan
}  // namespace mg

using namespace mg;

extern "C" size_t mg_scan_ckpt_elems(int B, int T, int Di) {
  if (B < 1 || T < 1 || Di < 1) return 0;
  return static_cast<size_t>((T + scan::kCkptRows - 1) / scan::kCkptRows) * B * Di;
}

extern "C" size_t mg_scan_workspace_bytes(int B, int T, int Di) {
  if (B < 1 || T < 1 || Di < 1) return 256;
  return scan::ws_bytes_any(B, T, Di);
}

extern "C" int mg_scan_workspace_init(void* workspace, size_t workspace_bytes, int B, int T, int Di, void* stream) {
  const char* fn = "mg_scan_workspace_init";
  if (B < 1 || T < 1 || Di < 4 || Di % scan::kVec) return fail(MG_ERR_ARG, "%s: bad shape B=%d T=%d Di=%d", fn, B, T, Di);
  const size_t need = scan::ws_bytes_any(B, T, Di);
  if (!workspace || workspace_bytes < need)
    return fail(MG_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", fn, workspace_bytes, need);
  if (!aligned(workspace, 16)) return fail(MG_ERR_ARG, "%s: workspace not 16-byte aligned", fn);
  const int64_t n16 = static_cast<int64_t>(need / 16);
  const int blocks = static_cast<int>(std::min<int64_t>((n16 + 255) / 256, 4096));
  hipLaunchKernelGGL(scan::init_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint4*>(workspace), n16, B, T, Di, scan::kDefaultPolls);
  return check_launch(fn);
}

extern "C" int mg_scan_workspace_set_max_polls(void* workspace, uint32_t max_polls, void* stream) {
  const char* fn = "mg_scan_workspace_set_max_polls";
  if (!workspace || !aligned(workspace, 16)) return fail(MG_ERR_ARG, "%s: bad workspace pointer", fn);
  if (max_polls < 1) return fail(MG_ERR_ARG, "%s: max_polls must be at least 1", fn);
  hipLaunchKernelGGL(scan::set_polls_kernel, dim3(1), dim3(1), 0, static_cast<hipStream_t>(stream),
                     scan::ws_header(workspace), max_polls);
  return check_launch(fn);
}

namespace mg {
namespace scan {
// The error of a header read back to the host (MG_OK when it is clean).
static int header_error(const char* fn, const WsHeader& h) {
  if (h.magic != kWsMagic) return fail(MG_ERR_WORKSPACE, "%s: workspace was never initialised", fn);
  if (h.err & kErrShape)
    return fail(MG_ERR_WORKSPACE, "%s: a scan call used this workspace (initialised for B=%d T=%d Di=%d) with "
                "another shape; its results are invalid", fn, h.B, h.T, h.Di);
  if (h.err & kErrStall)
    return fail(MG_ERR_STALL, "%s: a look-back wait gave up after %u polls%s (overlapping calls on one workspace, "
                "or a corrupted workspace); results invalid, initialise it again", fn, h.max_polls,
                (h.err & kErrTicket) ? " and a ticket past the last tile was drawn" : "");
  if (h.err & kErrTicket)
    return fail(MG_ERR_WORKSPACE, "%s: ticket counters corrupted (overlapping calls on one workspace?); results "
                "invalid, initialise it again", fn);
  return MG_OK;
}

// One thread: ORs the header's error bits (and kErrShape for a missing
// header) into a host word. Writes only when there is something to report.
__global__ void poll_kernel(const WsHeader* __restrict__ h, uint32_t* host_word) {
  uint32_t e = h->err;
  if (h->magic != kWsMagic) e |= kErrShape;
  if (e) *host_word = *host_word | e;
}
}  // namespace scan
}  // namespace mg

extern "C" int mg_scan_workspace_check(const void* workspace, void* stream) {
  const char* fn = "mg_scan_workspace_check";
  if (!workspace) return fail(MG_ERR_ARG, "%s: NULL workspace", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  scan::WsHeader h;
  hipError_t e = hipStreamSynchronize(st);
  if (e == hipSuccess) e = hipMemcpy(&h, workspace, sizeof(h), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return fail(MG_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
  return scan::header_error(fn, h);
}

extern "C" int mg_scan_workspace_poll(const void* workspace, uint32_t* host_word, void* stream) {
  const char* fn = "mg_scan_workspace_poll";
  if (!workspace || !aligned(workspace, 16)) return fail(MG_ERR_ARG, "%s: bad workspace pointer", fn);
  if (!host_word || !aligned(host_word, 4)) return fail(MG_ERR_ARG, "%s: bad host word pointer", fn);
  void* dev_word = nullptr;
  hipError_t e = hipHostGetDevicePointer(&dev_word, host_word, 0);
  if (e != hipSuccess || !dev_word)
    return fail(MG_ERR_ARG, "%s: host_word is not pinned host memory (hipHostGetDevicePointer: %s)", fn,
                hipGetErrorString(e));
  hipLaunchKernelGGL(scan::poll_kernel, dim3(1), dim3(1), 0, static_cast<hipStream_t>(stream),
                     static_cast<const scan::WsHeader*>(workspace), static_cast<uint32_t*>(dev_word));
  return check_launch(fn);
}

namespace mg {
namespace scan {
// Checks every argument of a forward call; need: the workspace bytes required
// (see check_common).
static int fwd_check(const char* fn, int in_dtype, const void* hidden, const void* gate, int64_t in_sb,
                     int64_t in_ld, const float* h0, int out_dtype, const void* h, int64_t out_sb, int64_t out_ld,
                     const float* h_last, const float* ckpt, int B, int T, int Di, void* workspace,
                     size_t workspace_bytes, size_t need, Geometry& g) {
  int rc;
  if ((rc = check_common(fn, B, T, Di, kFwdTileRows, workspace, workspace_bytes, g, need))) return rc;
  if ((rc = check_tensor(fn, "hidden", hidden, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = check_tensor(fn, "gate", gate, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = check_tensor(fn, "h", h, out_dtype, out_sb, out_ld))) return rc;
  if ((rc = check_f32vec(fn, "h0", h0))) return rc;
  if ((rc = check_f32vec(fn, "h_last", h_last))) return rc;
  if ((rc = check_f32vec(fn, "ckpt", ckpt))) return rc;
  if (!(in_dtype == MG_BF16 || (in_dtype == MG_F32 && out_dtype == MG_F32)))
    return fail(MG_ERR_DTYPE, "%s: in_dtype=%d out_dtype=%d unsupported", fn, in_dtype, out_dtype);
  return MG_OK;
}

// Launches a forward whose arguments fwd_check accepted.
static int fwd_launch(const char* fn, int in_dtype, const void* hidden, const void* gate, int64_t in_sb,
                      int64_t in_ld, const float* h0, int out_dtype, void* h, int64_t out_sb, int64_t out_ld,
                      float* h_last, float* ckpt, const Geometry& g, void* workspace, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == MG_BF16 && out_dtype == MG_BF16)
    launch_fwd<bf16_t, bf16_t>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, h_last, ckpt, g, workspace, st);
  else if (in_dtype == MG_F32)
    launch_fwd<float, float>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, h_last, ckpt, g, workspace, st);
  else
    launch_fwd<bf16_t, float>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, h_last, ckpt, g, workspace, st);
  return check_launch(fn);
}
}  // namespace scan
}  // namespace mg

extern "C" int mg_scan_fwd(int in_dtype, const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld,
                           const float* h0, int out_dtype, void* h, int64_t out_sb, int64_t out_ld,
                           float* h_last, float* ckpt, int B, int T, int Di, void* workspace,
                           size_t workspace_bytes, void* stream) {
  const char* fn = "mg_scan_fwd";
  scan::Geometry g;
  if (int rc = scan::fwd_check(fn, in_dtype, hidden, gate, in_sb, in_ld, h0, out_dtype, h, out_sb, out_ld, h_last,
                               ckpt, B, T, Di, workspace, workspace_bytes, 0, g))
    return rc;
  return scan::fwd_launch(fn, in_dtype, hidden, gate, in_sb, in_ld, h0, out_dtype, h, out_sb, out_ld, h_last, ckpt, g,
                          workspace, stream);
}

extern "C" int mg_scan_fwd_residual(int in_dtype, const void* hidden, const void* gate, int64_t in_sb,
                                    int64_t in_ld, const float* h0, const float* res, float* x_out, int64_t out_sb,
                                    int64_t out_ld, float* h_last, float* ckpt, int B, int T, int Di,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "mg_scan_fwd_residual";
  scan::Geometry g;
  if (!ckpt) return fail(MG_ERR_ARG, "%s: ckpt is required (the backward rebuilds h from it)", fn);
  if (int rc = scan::check_tensor(fn, "res", res, MG_F32, out_sb, out_ld)) return rc;
  if (int rc = scan::fwd_check(fn, in_dtype, hidden, gate, in_sb, in_ld, h0, MG_F32, x_out, out_sb, out_ld, h_last,
                               ckpt, B, T, Di, workspace, workspace_bytes, 0, g))
    return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == MG_F32)
    scan::launch_fwd<float, float>(hidden, gate, in_sb, in_ld, h0, x_out, out_sb, out_ld, h_last, ckpt, g, workspace,
                                   st, res);
  else
    scan::launch_fwd<bf16_t, float>(hidden, gate, in_sb, in_ld, h0, x_out, out_sb, out_ld, h_last, ckpt, g,
                                    workspace, st, res);
  return check_launch(fn);
}

extern "C" size_t mg_scan_fwd_noalloc_max_bytes(void) { return scan::kNoAllocBytes; }

extern "C" int mg_scan_fwd_noalloc(int in_dtype, const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld,
                                   const float* h0, int out_dtype, void* h, int64_t out_sb, int64_t out_ld,
                                   float* h_last, float* ckpt, int B, int T, int Di, void* stream) {
  const char* fn = "mg_scan_fwd_noalloc";
  if (B < 1 || T < 1 || Di < 4 || Di % scan::kVec) return fail(MG_ERR_ARG, "%s: bad shape B=%d T=%d Di=%d", fn, B, T, Di);
  const size_t need = scan::fwd_ws_bytes(B, T, Di);
  if (need > scan::kNoAllocBytes)
    return fail(MG_ERR_ARG, "%s: B=%d T=%d Di=%d needs %zu bytes of look-back scratch, above the allocation-free "
                "maximum of %zu (use mg_scan_fwd with a workspace)", fn, B, T, Di, need, scan::kNoAllocBytes);
  void* ws = nullptr;
  if (int rc = scan::scratch_ptr(fn, &ws)) return rc;
  // every argument is checked before anything is enqueued: a rejected call
  // leaves the scratch (and any call still running on it) alone
  scan::Geometry g;
  if (int rc = scan::fwd_check(fn, in_dtype, hidden, gate, in_sb, in_ld, h0, out_dtype, h, out_sb, out_ld, h_last,
                               ckpt, B, T, Di, ws, scan::kNoAllocBytes, need, g))
    return rc;
  // initialise the part this call uses (zeros + header), then the forward on it
  const int64_t n16 = static_cast<int64_t>((need + 15) / 16);
  const int blocks = static_cast<int>(std::min<int64_t>((n16 + 255) / 256, 4096));
  hipLaunchKernelGGL(scan::init_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint4*>(ws), n16, B, T, Di, scan::kDefaultPolls);
  if (int rc = check_launch(fn)) return rc;
  return scan::fwd_launch(fn, in_dtype, hidden, gate, in_sb, in_ld, h0, out_dtype, h, out_sb, out_ld, h_last, ckpt, g,
                          ws, stream);
}

extern "C" int mg_scan_fwd_noalloc_check(void* stream) {
  const char* fn = "mg_scan_fwd_noalloc_check";
  void* ws = nullptr;
  if (int rc = scan::scratch_ptr(fn, &ws)) return rc;
  scan::WsHeader h;
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e == hipSuccess) e = hipMemcpy(&h, ws, sizeof(h), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return fail(MG_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
  return scan::header_error(fn, h);
}

extern "C" int mg_scan_bwd(int in_dtype, const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld,
                           const float* h0, int out_dtype, const void* h, int64_t out_sb, int64_t out_ld,
                           const float* ckpt, const void* dh, int64_t g_sb, int64_t g_ld, const float* dh_last,
                           void* dhidden, void* dgate, int64_t d_sb, int64_t d_ld, float* dh0, int B, int T, int Di,
                           void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "mg_scan_bwd";
  scan::Geometry g;
  int rc;
  if ((rc = scan::check_common(fn, B, T, Di, scan::kBwdTileRows, workspace, workspace_bytes, g))) return rc;
  if ((rc = scan::check_tensor(fn, "hidden", hidden, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "gate", gate, in_dtype, in_sb, in_ld))) return rc;
  if (!(h == nullptr && ckpt) && (rc = scan::check_tensor(fn, "h", h, out_dtype, out_sb, out_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "dh", dh, out_dtype, g_sb, g_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "dhidden", dhidden, in_dtype, d_sb, d_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "dgate", dgate, in_dtype, d_sb, d_ld))) return rc;
  if ((rc = scan::check_f32vec(fn, "h0", h0))) return rc;
  if ((rc = scan::check_f32vec(fn, "dh_last", dh_last))) return rc;
  if ((rc = scan::check_f32vec(fn, "dh0", dh0))) return rc;
  if ((rc = scan::check_f32vec(fn, "ckpt", ckpt))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == MG_BF16 && out_dtype == MG_BF16)
    scan::launch_bwd<bf16_t, bf16_t>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, ckpt, dh, g_sb, g_ld, dh_last,
                                     dhidden, dgate, d_sb, d_ld, dh0, g, workspace, st);
  else if (in_dtype == MG_F32 && out_dtype == MG_F32)
    scan::launch_bwd<float, float>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, ckpt, dh, g_sb, g_ld, dh_last,
                                   dhidden, dgate, d_sb, d_ld, dh0, g, workspace, st);
  else if (in_dtype == MG_BF16 && out_dtype == MG_F32)
    scan::launch_bwd<bf16_t, float>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, ckpt, dh, g_sb, g_ld, dh_last,
                                    dhidden, dgate, d_sb, d_ld, dh0, g, workspace, st);
  else
    return fail(MG_ERR_DTYPE, "%s: in_dtype=%d out_dtype=%d unsupported", fn, in_dtype, out_dtype);
  return check_launch(fn);
}
