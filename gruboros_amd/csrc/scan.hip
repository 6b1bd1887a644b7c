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
//   * A tile is kTileRows consecutive time steps x kTileCh consecutive
//     channels of one batch row; one 256-thread workgroup per tile.
//   * Thread (cl, s) owns 4 adjacent channels (one 8-byte bf16 / 16-byte
//     fp32 vector per row) and a run of kSubRows consecutive time steps.
//     16 lanes cover 64 channels, so every row segment a wave touches is a
//     full 128-byte line for bf16.
//   * Each thread scans its run in registers and produces the run's affine
//     map h -> A h + V. Runs are combined in LDS; the tile's map is handed
//     to later tiles through look-back words in the workspace (decoupled
//     look-back). Tiles take tickets from an atomic counter so a tile only
//     ever waits on tiles that were started before it.
//   * The backward walks tiles in reverse time order. It needs h_{t-1};
//     instead of reading the forward output it rebuilds h in fp32 from the
//     per-tile entry state the forward saved (ckpt), which saves 2 bytes per
//     element of traffic and keeps h at fp32 accuracy for bf16 outputs.

#include <algorithm>

#include "mg_common.h"

namespace mg {
namespace scan {

constexpr int kVec = 4;                       // channels per thread
constexpr int kChLanes = 16;                  // threads across channels
constexpr int kSubs = 16;                     // time runs per tile
constexpr int kSubRows = 8;                   // time steps per run
constexpr int kThreads = kChLanes * kSubs;    // 256
constexpr int kTileRows = kSubs * kSubRows;   // 128
constexpr int kTileCh = kChLanes * kVec;      // 64
constexpr size_t kWsHeader = 256;             // ticket counter lives here

struct Geometry {
  int B, T, Di;
  int nblk_d;   // channel blocks per batch row
  int ncb;      // channel blocks in total (B * nblk_d)
  int ntiles;   // time tiles
  int64_t BD;   // B * Di
};

__device__ __forceinline__ void tile_coords(const Geometry& g, uint32_t ticket, bool reverse,
                                            int& k, int& b, int& d) {
  const int kk = static_cast<int>(ticket / g.ncb);
  const int cbi = static_cast<int>(ticket % g.ncb);
  k = reverse ? (g.ntiles - 1 - kk) : kk;
  b = cbi / g.nblk_d;
  d = (cbi % g.nblk_d) * kTileCh + (static_cast<int>(threadIdx.x) % kChLanes) * kVec;
}

// Walk back (forward scan: towards earlier tiles, step = -1; backward scan:
// towards later tiles, step = +1) until an inclusive prefix is found, folding
// aggregates on the way. Returns the state entering tile k for 4 channels.
__device__ __forceinline__ f4 look_back(const uint64_t* status, int64_t BD, int64_t c, int k, int step) {
  float accA[kVec], accV[kVec], carry[kVec];
  int kk[kVec];
  unsigned done = 0;
#pragma unroll
  for (int j = 0; j < kVec; ++j) { accA[j] = 1.0f; accV[j] = 0.0f; carry[j] = 0.0f; kk[j] = k + step; }
  while (done != (1u << kVec) - 1u) {
    uint64_t w[kVec];
#pragma unroll
    for (int j = 0; j < kVec; ++j)
      w[j] = (done >> j) & 1u ? 0ull : poll_word(status + static_cast<int64_t>(kk[j]) * BD + c + j);
    bool progress = false;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      if ((done >> j) & 1u) continue;
      const uint32_t tag = static_cast<uint32_t>(w[j]);
      const float val = __uint_as_float(static_cast<uint32_t>(w[j] >> 32));
      if (tag == kTagIncl) {
        carry[j] = accA[j] * val + accV[j];
        done |= 1u << j;
        progress = true;
      } else if (tag & kTagAggBit) {
        const float Aj = __uint_as_float(tag & ~kTagAggBit);
        accV[j] = accA[j] * val + accV[j];
        accA[j] = accA[j] * Aj;
        kk[j] += step;
        progress = true;
      }
    }
    if (!progress) __builtin_amdgcn_s_sleep(2);
  }
  return f4{{carry[0], carry[1], carry[2], carry[3]}};
}

// ------------------------------------------------------------------ forward

template <typename Tin, typename Tout>
__global__ __launch_bounds__(kThreads) void scan_fwd_kernel(
    const Tin* __restrict__ hidden, const Tin* __restrict__ gate, int64_t in_sb, int64_t in_ld,
    const float* __restrict__ h0, Tout* __restrict__ hout, int64_t out_sb, int64_t out_ld,
    float* __restrict__ h_last, float* __restrict__ ckpt, Geometry g,
    uint32_t* __restrict__ counter, uint64_t* __restrict__ status) {
  __shared__ uint32_t s_ticket;
  __shared__ f4 s_A[kSubs][kChLanes];
  __shared__ f4 s_V[kSubs][kChLanes];
  __shared__ f4 s_carry[kChLanes];

  const int tid = threadIdx.x;
  const int cl = tid % kChLanes;
  const int s = tid / kChLanes;
  if (tid == 0) s_ticket = atomicAdd(counter, 1u);
  __syncthreads();
  int k, b, d;
  tile_coords(g, s_ticket, false, k, b, d);
  const bool ok = d < g.Di;
  const int t0 = k * kTileRows + s * kSubRows;
  const int64_t c = static_cast<int64_t>(b) * g.Di + d;

  // Load the run (all loads issued before any math).
  f4 hv[kSubRows] = {}, gv[kSubRows] = {};
  const Tin* hp = hidden + b * in_sb + static_cast<int64_t>(t0) * in_ld + d;
  const Tin* gp = gate + b * in_sb + static_cast<int64_t>(t0) * in_ld + d;
#pragma unroll
  for (int i = 0; i < kSubRows; ++i) {
    if (ok && t0 + i < g.T) {
      hv[i] = io4<Tin>::load(hp + i * in_ld);
      gv[i] = io4<Tin>::load(gp + i * in_ld);
    }
  }

  // a_t, v_t = z_t g(hidden_t); rows past T are the identity map.
  float a[kSubRows][kVec], v[kSubRows][kVec];
  f4 A, V;
#pragma unroll
  for (int j = 0; j < kVec; ++j) { A.v[j] = 1.0f; V.v[j] = 0.0f; }
#pragma unroll
  for (int i = 0; i < kSubRows; ++i) {
    const bool live = ok && t0 + i < g.T;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      float aa, zz;
      gate_coeffs(gv[i].v[j], aa, zz);
      a[i][j] = live ? aa : 1.0f;
      v[i][j] = live ? zz * g_tilde(hv[i].v[j]) : 0.0f;
      V.v[j] = a[i][j] * V.v[j] + v[i][j];
      A.v[j] = A.v[j] * a[i][j];
    }
  }
  s_A[s][cl] = A;
  s_V[s][cl] = V;
  __syncthreads();

  if (s == 0 && ok) {
    f4 TA, TV;
#pragma unroll
    for (int j = 0; j < kVec; ++j) { TA.v[j] = 1.0f; TV.v[j] = 0.0f; }
    for (int q = 0; q < kSubs; ++q) {
      const f4 qa = s_A[q][cl], qv = s_V[q][cl];
#pragma unroll
      for (int j = 0; j < kVec; ++j) { TV.v[j] = qa.v[j] * TV.v[j] + qv.v[j]; TA.v[j] *= qa.v[j]; }
    }
    uint64_t* st = status + static_cast<int64_t>(k) * g.BD + c;
    f4 carry;
    if (k == 0) {
      if (h0) carry = io4<float>::load(h0 + c);
      else { for (int j = 0; j < kVec; ++j) carry.v[j] = 0.0f; }
    } else {
#pragma unroll
      for (int j = 0; j < kVec; ++j) publish_agg(st + j, TA.v[j], TV.v[j]);
      carry = look_back(status, g.BD, c, k, -1);
    }
    if (k + 1 < g.ntiles) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) publish_incl(st + j, TA.v[j] * carry.v[j] + TV.v[j]);
    }
    s_carry[cl] = carry;
    if (ckpt) io4<float>::store(ckpt + static_cast<int64_t>(k) * g.BD + c, carry);
  }
  __syncthreads();
  if (!ok) return;

  // State entering this run, then replay it.
  f4 h = s_carry[cl];
  for (int q = 0; q < s; ++q) {
    const f4 qa = s_A[q][cl], qv = s_V[q][cl];
#pragma unroll
    for (int j = 0; j < kVec; ++j) h.v[j] = qa.v[j] * h.v[j] + qv.v[j];
  }
  Tout* op = hout + b * out_sb + static_cast<int64_t>(t0) * out_ld + d;
#pragma unroll
  for (int i = 0; i < kSubRows; ++i) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) h.v[j] = a[i][j] * h.v[j] + v[i][j];
    if (t0 + i < g.T) io4<Tout>::store(op + i * out_ld, h);
    if (h_last && t0 + i == g.T - 1) io4<float>::store(h_last + c, h);
  }
}

// ------------------------------------------------------------------ backward

template <typename Tin, typename Tg>
__global__ __launch_bounds__(kThreads) void scan_bwd_kernel(
    const Tin* __restrict__ hidden, const Tin* __restrict__ gate, int64_t in_sb, int64_t in_ld,
    const float* __restrict__ ckpt, const Tg* __restrict__ dh, int64_t g_sb, int64_t g_ld,
    const float* __restrict__ dh_last, Tin* __restrict__ dhidden, Tin* __restrict__ dgate,
    float* __restrict__ dh0, Geometry g, uint32_t* __restrict__ counter,
    uint64_t* __restrict__ status) {
  __shared__ uint32_t s_ticket;
  __shared__ f4 s_A[kSubs][kChLanes];
  __shared__ f4 s_V[kSubs][kChLanes];
  __shared__ f4 s_carry[kChLanes];

  const int tid = threadIdx.x;
  const int cl = tid % kChLanes;
  const int s = tid / kChLanes;
  if (tid == 0) s_ticket = atomicAdd(counter, 1u);
  __syncthreads();
  int k, b, d;
  tile_coords(g, s_ticket, true, k, b, d);
  const bool ok = d < g.Di;
  const int t0 = k * kTileRows + s * kSubRows;
  const int64_t c = static_cast<int64_t>(b) * g.Di + d;

  f4 hv[kSubRows] = {}, gv[kSubRows] = {}, dv[kSubRows] = {};
  const int64_t in_off = b * in_sb + static_cast<int64_t>(t0) * in_ld + d;
  const Tin* hp = hidden + in_off;
  const Tin* gp = gate + in_off;
  const Tg* dp = dh + b * g_sb + static_cast<int64_t>(t0) * g_ld + d;
#pragma unroll
  for (int i = 0; i < kSubRows; ++i) {
    if (ok && t0 + i < g.T) {
      hv[i] = io4<Tin>::load(hp + i * in_ld);
      gv[i] = io4<Tin>::load(gp + i * in_ld);
      dv[i] = io4<Tg>::load(dp + i * g_ld);
    }
  }
  f4 hc = {};  // state entering the tile (saved by the forward)
  if (ok) hc = io4<float>::load(ckpt + static_cast<int64_t>(k) * g.BD + c);
  if (ok && dh_last && t0 <= g.T - 1 && g.T - 1 < t0 + kSubRows) {
    const f4 dl = io4<float>::load(dh_last + c);
    const int i = g.T - 1 - t0;
#pragma unroll
    for (int ii = 0; ii < kSubRows; ++ii)
      if (ii == i) {
#pragma unroll
        for (int j = 0; j < kVec; ++j) dv[ii].v[j] += dl.v[j];
      }
  }

  // Per element: a (recurrence coefficient), v = z g~ (forward input),
  // z, q = z g'(hidden), gh (incoming gradient). v and z are folded into
  // dgate's factor once h_{t-1} is known.
  float a[kSubRows][kVec], v[kSubRows][kVec], z[kSubRows][kVec], q[kSubRows][kVec], gh[kSubRows][kVec];
  f4 A, V;
#pragma unroll
  for (int j = 0; j < kVec; ++j) { A.v[j] = 1.0f; V.v[j] = 0.0f; }
#pragma unroll
  for (int i = 0; i < kSubRows; ++i) {
    const bool live = ok && t0 + i < g.T;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      float aa, zz, gt, gp_;
      gate_coeffs(gv[i].v[j], aa, zz);
      g_tilde_grad(hv[i].v[j], gt, gp_);
      a[i][j] = live ? aa : 1.0f;
      z[i][j] = live ? zz : 0.0f;
      v[i][j] = live ? zz * gt : 0.0f;
      q[i][j] = live ? zz * gp_ : 0.0f;
      gh[i][j] = live ? dv[i].v[j] : 0.0f;
      V.v[j] = a[i][j] * V.v[j] + v[i][j];
      A.v[j] = A.v[j] * a[i][j];
    }
  }
  s_A[s][cl] = A;
  s_V[s][cl] = V;
  __syncthreads();

  // Rebuild h_{t-1} for the run; keep dgate's factor a z (g~ - h_{t-1})
  // = a (v - z h_{t-1}) in v.
  if (ok) {
    for (int qq = 0; qq < s; ++qq) {
      const f4 qa = s_A[qq][cl], qv = s_V[qq][cl];
#pragma unroll
      for (int j = 0; j < kVec; ++j) hc.v[j] = qa.v[j] * hc.v[j] + qv.v[j];
    }
  }
#pragma unroll
  for (int i = 0; i < kSubRows; ++i) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const float hprev = hc.v[j];
      hc.v[j] = a[i][j] * hprev + v[i][j];
      v[i][j] = a[i][j] * (v[i][j] - z[i][j] * hprev);
    }
  }

  // Reverse run map mu -> A mu + M with mu_t = a_t lambda_t,
  // lambda_t = gh_t + mu_{t+1}.
  f4 M;
#pragma unroll
  for (int j = 0; j < kVec; ++j) { A.v[j] = 1.0f; M.v[j] = 0.0f; }
#pragma unroll
  for (int i = kSubRows - 1; i >= 0; --i) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      M.v[j] = a[i][j] * (gh[i][j] + M.v[j]);
      A.v[j] = A.v[j] * a[i][j];
    }
  }
  __syncthreads();  // forward run maps no longer needed
  s_A[s][cl] = A;
  s_V[s][cl] = M;
  __syncthreads();

  if (s == 0 && ok) {
    f4 TA, TM;
#pragma unroll
    for (int j = 0; j < kVec; ++j) { TA.v[j] = 1.0f; TM.v[j] = 0.0f; }
    for (int qq = kSubs - 1; qq >= 0; --qq) {
      const f4 qa = s_A[qq][cl], qm = s_V[qq][cl];
#pragma unroll
      for (int j = 0; j < kVec; ++j) { TM.v[j] = qa.v[j] * TM.v[j] + qm.v[j]; TA.v[j] *= qa.v[j]; }
    }
    uint64_t* st = status + static_cast<int64_t>(k) * g.BD + c;
    f4 carry;
    if (k == g.ntiles - 1) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) carry.v[j] = 0.0f;
    } else {
#pragma unroll
      for (int j = 0; j < kVec; ++j) publish_agg(st + j, TA.v[j], TM.v[j]);
      carry = look_back(status, g.BD, c, k, +1);
    }
    if (k > 0) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) publish_incl(st + j, TA.v[j] * carry.v[j] + TM.v[j]);
    }
    s_carry[cl] = carry;
  }
  __syncthreads();
  if (!ok) return;

  f4 mu = s_carry[cl];
  for (int qq = kSubs - 1; qq > s; --qq) {
    const f4 qa = s_A[qq][cl], qm = s_V[qq][cl];
#pragma unroll
    for (int j = 0; j < kVec; ++j) mu.v[j] = qa.v[j] * mu.v[j] + qm.v[j];
  }
  Tin* dhp = dhidden + in_off;
  Tin* dgp = dgate + in_off;
#pragma unroll
  for (int i = kSubRows - 1; i >= 0; --i) {
    f4 og, oh;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const float lam = gh[i][j] + mu.v[j];
      og.v[j] = lam * v[i][j];
      oh.v[j] = lam * q[i][j];
      mu.v[j] = a[i][j] * lam;
    }
    if (t0 + i < g.T) {
      io4<Tin>::store(dgp + i * in_ld, og);
      io4<Tin>::store(dhp + i * in_ld, oh);
    }
  }
  if (dh0 && t0 == 0) io4<float>::store(dh0 + c, mu);
}

// ------------------------------------------------------------------ host

__global__ void zero_kernel(uint4* __restrict__ p, int64_t n16) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

inline size_t ws_bytes(int B, int T, int Di) {
  const int nt = (T + kTileRows - 1) / kTileRows;
  return kWsHeader + static_cast<size_t>(nt) * B * Di * sizeof(uint64_t);
}

inline int check_common(const char* fn, int B, int T, int Di, void* ws, size_t ws_size,
                        Geometry& g) {
  if (B < 1 || T < 1 || Di < 4) return fail(MG_ERR_ARG, "%s: bad shape B=%d T=%d Di=%d", fn, B, T, Di);
  if (Di % kVec) return fail(MG_ERR_ARG, "%s: Di=%d must be a multiple of 4", fn, Di);
  const size_t need = ws_bytes(B, T, Di);
  if (!ws || ws_size < need)
    return fail(MG_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", fn, ws_size, need);
  if (!aligned(ws, 16)) return fail(MG_ERR_ARG, "%s: workspace not 16-byte aligned", fn);
  g.B = B; g.T = T; g.Di = Di;
  g.nblk_d = (Di + kTileCh - 1) / kTileCh;
  g.ncb = B * g.nblk_d;
  g.ntiles = (T + kTileRows - 1) / kTileRows;
  g.BD = static_cast<int64_t>(B) * Di;
  const int64_t nblocks = static_cast<int64_t>(g.ncb) * g.ntiles;
  if (nblocks > 0x7fffffff) return fail(MG_ERR_ARG, "%s: problem too large (%lld tiles)", fn, (long long)nblocks);
  return MG_OK;
}

inline int check_tensor(const char* fn, const char* name, const void* p, int dtype, int64_t sb, int64_t ld) {
  if (!p) return fail(MG_ERR_ARG, "%s: %s is NULL", fn, name);
  if (dtype != MG_F32 && dtype != MG_BF16) return fail(MG_ERR_DTYPE, "%s: %s dtype %d unsupported", fn, name, dtype);
  if (sb % kVec || ld % kVec || sb < 0 || ld < 0)
    return fail(MG_ERR_ARG, "%s: %s strides (%lld, %lld) must be non-negative multiples of 4", fn, name,
                (long long)sb, (long long)ld);
  if (!aligned(p, dtype == MG_F32 ? 16 : 8)) return fail(MG_ERR_ARG, "%s: %s misaligned", fn, name);
  return MG_OK;
}

inline int check_f32vec(const char* fn, const char* name, const void* p) {
  if (p && !aligned(p, 16)) return fail(MG_ERR_ARG, "%s: %s not 16-byte aligned", fn, name);
  return MG_OK;
}

inline void zero_ws(void* ws, const Geometry& g, hipStream_t st) {
  const int64_t n16 = static_cast<int64_t>(ws_bytes(g.B, g.T, g.Di) / 16);
  const int blocks = static_cast<int>(std::min<int64_t>((n16 + 255) / 256, 4096));
  hipLaunchKernelGGL(zero_kernel, dim3(blocks), dim3(256), 0, st, static_cast<uint4*>(ws), n16);
}

template <typename Tin, typename Tout>
void launch_fwd(const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld, const float* h0, void* h,
                int64_t out_sb, int64_t out_ld, float* h_last, float* ckpt, const Geometry& g, void* ws,
                hipStream_t st) {
  auto* counter = static_cast<uint32_t*>(ws);
  auto* status = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + kWsHeader);
  hipLaunchKernelGGL((scan_fwd_kernel<Tin, Tout>), dim3(g.ncb * g.ntiles), dim3(kThreads), 0, st,
                     static_cast<const Tin*>(hidden), static_cast<const Tin*>(gate), in_sb, in_ld, h0,
                     static_cast<Tout*>(h), out_sb, out_ld, h_last, ckpt, g, counter, status);
}

template <typename Tin, typename Tg>
void launch_bwd(const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld, const float* ckpt,
                const void* dh, int64_t g_sb, int64_t g_ld, const float* dh_last, void* dhidden, void* dgate,
                float* dh0, const Geometry& g, void* ws, hipStream_t st) {
  auto* counter = static_cast<uint32_t*>(ws);
  auto* status = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + kWsHeader);
  hipLaunchKernelGGL((scan_bwd_kernel<Tin, Tg>), dim3(g.ncb * g.ntiles), dim3(kThreads), 0, st,
                     static_cast<const Tin*>(hidden), static_cast<const Tin*>(gate), in_sb, in_ld, ckpt,
                     static_cast<const Tg*>(dh), g_sb, g_ld, dh_last, static_cast<Tin*>(dhidden),
                     static_cast<Tin*>(dgate), dh0, g, counter, status);
}

}  // namespace scan
}  // namespace mg

using namespace mg;

extern "C" int mg_scan_num_tiles(int T) { return T < 1 ? 0 : (T + scan::kTileRows - 1) / scan::kTileRows; }

extern "C" size_t mg_scan_workspace_bytes(int B, int T, int Di) {
  if (B < 1 || T < 1 || Di < 1) return scan::kWsHeader;
  return scan::ws_bytes(B, T, Di);
}

extern "C" int mg_scan_fwd(int in_dtype, const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld,
                           const float* h0, int out_dtype, void* h, int64_t out_sb, int64_t out_ld,
                           float* h_last, float* ckpt, int B, int T, int Di, void* workspace,
                           size_t workspace_bytes, void* stream) {
  const char* fn = "mg_scan_fwd";
  scan::Geometry g;
  int rc;
  if ((rc = scan::check_common(fn, B, T, Di, workspace, workspace_bytes, g))) return rc;
  if ((rc = scan::check_tensor(fn, "hidden", hidden, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "gate", gate, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "h", h, out_dtype, out_sb, out_ld))) return rc;
  if ((rc = scan::check_f32vec(fn, "h0", h0))) return rc;
  if ((rc = scan::check_f32vec(fn, "h_last", h_last))) return rc;
  if ((rc = scan::check_f32vec(fn, "ckpt", ckpt))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  scan::zero_ws(workspace, g, st);
  if (in_dtype == MG_BF16 && out_dtype == MG_BF16)
    scan::launch_fwd<bf16_t, bf16_t>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, h_last, ckpt, g, workspace, st);
  else if (in_dtype == MG_F32 && out_dtype == MG_F32)
    scan::launch_fwd<float, float>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, h_last, ckpt, g, workspace, st);
  else if (in_dtype == MG_BF16 && out_dtype == MG_F32)
    scan::launch_fwd<bf16_t, float>(hidden, gate, in_sb, in_ld, h0, h, out_sb, out_ld, h_last, ckpt, g, workspace, st);
  else
    return fail(MG_ERR_DTYPE, "%s: in_dtype=%d out_dtype=%d unsupported", fn, in_dtype, out_dtype);
  return check_launch(fn);
}

extern "C" int mg_scan_bwd(int in_dtype, const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld,
                           const float* h0, const float* ckpt, int g_dtype, const void* dh, int64_t g_sb,
                           int64_t g_ld, const float* dh_last, void* dhidden, void* dgate, float* dh0, int B,
                           int T, int Di, void* workspace, size_t workspace_bytes, void* stream) {
  (void)h0;  // the entry state of tile 0 (h0 or 0) is already in ckpt
  const char* fn = "mg_scan_bwd";
  scan::Geometry g;
  int rc;
  if ((rc = scan::check_common(fn, B, T, Di, workspace, workspace_bytes, g))) return rc;
  if ((rc = scan::check_tensor(fn, "hidden", hidden, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "gate", gate, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "dh", dh, g_dtype, g_sb, g_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "dhidden", dhidden, in_dtype, in_sb, in_ld))) return rc;
  if ((rc = scan::check_tensor(fn, "dgate", dgate, in_dtype, in_sb, in_ld))) return rc;
  if (!ckpt) return fail(MG_ERR_ARG, "%s: ckpt is NULL (run mg_scan_fwd with ckpt first)", fn);
  if ((rc = scan::check_f32vec(fn, "ckpt", ckpt))) return rc;
  if ((rc = scan::check_f32vec(fn, "dh_last", dh_last))) return rc;
  if ((rc = scan::check_f32vec(fn, "dh0", dh0))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  scan::zero_ws(workspace, g, st);
  if (in_dtype == MG_BF16 && g_dtype == MG_BF16)
    scan::launch_bwd<bf16_t, bf16_t>(hidden, gate, in_sb, in_ld, ckpt, dh, g_sb, g_ld, dh_last, dhidden, dgate, dh0, g, workspace, st);
  else if (in_dtype == MG_F32 && g_dtype == MG_F32)
    scan::launch_bwd<float, float>(hidden, gate, in_sb, in_ld, ckpt, dh, g_sb, g_ld, dh_last, dhidden, dgate, dh0, g, workspace, st);
  else if (in_dtype == MG_BF16 && g_dtype == MG_F32)
    scan::launch_bwd<bf16_t, float>(hidden, gate, in_sb, in_ld, ckpt, dh, g_sb, g_ld, dh_last, dhidden, dgate, dh0, g, workspace, st);
  else
    return fail(MG_ERR_DTYPE, "%s: in_dtype=%d g_dtype=%d unsupported", fn, in_dtype, g_dtype);
  return check_launch(fn);
}
