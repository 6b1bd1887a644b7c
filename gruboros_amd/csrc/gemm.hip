// bf16 matrix products on MFMA (v_mfma_f32_32x32x16_bf16) with fp32
// accumulation, for the dense layers of the minLM step:
//   to_hidden_and_gate      reference mingru/minGRU.py:45   (Y = X W^T)
//   to_out                  reference mingru/minGRU.py:71
//   FeedForward             reference mingru/minLM.py:17-23 (Linear, GELU, Linear)
//   to_logits               reference mingru/minLM.py:75,138
// and their backward products (dX = dY W, dW = dY^T X).
//
// C[m, n] = sum_k A(m, k) B(k, n) with each operand in one of two layouts:
//   K-contiguous : element (row, k) at p + row * ld + k    (X, W as stored)
//   MN-contiguous: element (row, k) at p + k * ld + row    (dY^T, X^T for dW)
// The weight of Y = X W^T is the K-contiguous B (rows = output features).
//
// Workgroup tile BM x BN x 64 (BM, BN in {128, 256}), waves in a WM x WN
// grid, each owning (BM/WM) x (BN/WN) as 32 x 32 MFMA blocks. Operand tiles
// go from memory straight into LDS (buffer_load ... lds), two stages: the
// loads of tile k+1 are in flight while tile k is multiplied. K-contiguous
// tiles sit in LDS as [row][64 k] (128-byte rows, 16-byte chunk c of row r
// at chunk c ^ ((r ^ (r >> 3)) & 7)) and a fragment is one 16-byte LDS
// read; MN-contiguous tiles stay [64 k][rows] and their fragments come
// through the LDS transpose read (two 8-byte reads).
// Main loops (measured on MI355X):
//   mainloop_w8  256 x 256, eight waves (two per SIMD, 64 x 128 each), any
//                layout without masking (K % 64 == 0 for a K-contiguous
//                operand, a multiple of 256 rows for an MN-contiguous one):
//                every product of the cfg3 step, except the GELU-gradient
//                epilogue, which runs
//   mainloop_w4  the same pipeline with four waves of 128 x 128;
//   mainloop     masked tiles of other shapes, one barrier per k-tile, the
//                fragments of the next k-step read under the MFMAs of the
//                current one;
//   mainloop_pp  masked 256 x 256 with an MN-contiguous B: two wave groups
//                alternate between reading a whole k-tile of fragments and
//                multiplying it, a barrier between phases.
//
// The MFMA is fed the B fragment as its first operand and the A fragment as
// its second, so a lane's accumulator holds C[m][n..n+3] (4 consecutive
// output columns of one row) and stores are 8- or 16-byte vectors.
//
// Epilogues (fused into the store):
//   NONE       C = acc
//   BIAS       C = acc + bias[n]
//   BIAS_GELU  aux = bf16(acc + bias[n]);  C = gelu(aux)      (FeedForward up)
//   GELU_GRAD  C = acc * gelu'(aux[m][n])                     (its backward)
// with gelu(x) = x/2 (1 + erf(x / sqrt 2)), the exact form of nn.GELU().
// fp32 outputs may be split along K over several workgroups: each writes its
// partial tile to a workspace, and a second kernel adds the partials in split
// order into C, so the result does not depend on scheduling.
//
// Hi/lo products (MG_GEMM_HILO): each operand row holds K bf16 "hi" values
// followed by K bf16 "lo" values (x = hi + lo to ~2^-16 relative), and the
// k-loop runs three K segments, A_hi B_hi + A_lo B_hi + A_hi B_lo, into the
// same fp32 accumulators: an fp32-accurate product (the dropped A_lo B_lo
// term is ~2^-16 relative) at three times the MFMA work.

#include <algorithm>
#include <type_traits>
#include <utility>

#include "mg_common.h"

namespace mg {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;

struct Params {
  const bf16_t* A;
  const bf16_t* B;
  void* C;
  const float* bias;
  bf16_t* aux;
  int64_t lda, ldb, ldc, ldaux;
  int M, N, K;
  int tiles_m, tiles_n;
  int kt_per_split;  // k-tiles per split
  float* part;       // split partials: one dense [M, N] fp32 slice per split
  int xcd_splits;    // > 0: a 1-D grid of tiles x xcd_splits workgroups, laid out by split_tile_of
  int accumulate;    // C += (fp32 outputs)
  uint32_t a_span, b_span;  // bytes from A / B to one past their last element
  uint32_t aux_span;        // bytes of aux (GELU gradient's pre-activations)
  int hilo;                 // 1: hi/lo operands, three K segments of nkt_seg k-tiles
  int nkt_seg;              // k-tiles per K segment (ceil(K / 64))
  int hilo_cols;            // persistent four-wave kernel only, > 0: only output columns below
                            // it are hi/lo products, the rest take the hi halves' product alone
};

// k-tiles of the whole k-loop (three segments for hi/lo products)
__device__ __host__ __forceinline__ int total_ktiles(const Params& p) {
  return p.hilo ? 3 * p.nkt_seg : (p.K + BK - 1) / BK;
}

// Where global k-tile tg reads: first k within the segment, the mask bound
// (0 past kt1: those loads read zero) and the column offsets of A and B.
struct KTile {
  int k0, kmax, aofs, bofs;
};
__device__ __forceinline__ KTile ktile(const Params& p, int tg, int kt1) {
  KTile r;
  if (p.hilo) {
    const int seg = tg / p.nkt_seg;
    r.k0 = (tg - seg * p.nkt_seg) * BK;
    r.kmax = tg < kt1 ? p.K : 0;
    r.aofs = seg == 1 ? p.K : 0;
    r.bofs = seg == 2 ? p.K : 0;
  } else {
    r.k0 = tg * BK;
    r.kmax = min(p.K, kt1 * BK);
    r.aofs = r.bofs = 0;
  }
  return r;
}

__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r ^ (r >> 3)) & 7); }

// Operand tile loader: R rows x 64 k, into LDS as [R][8 chunks of 8 bf16].
// Global reads go through a buffer resource spanning exactly the operand, so
// rows (K-contiguous) or k-rows (MN-contiguous) past the end read as zero
// without branches; the contiguous dimension is masked with a select.
struct Operand {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t ld2;  // leading dimension in bytes
};

__device__ __forceinline__ Operand make_operand(const bf16_t* p, int64_t ld, uint32_t span_bytes) {
  Operand o;
  o.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(p), static_cast<short>(0),
                                             static_cast<int>(span_bytes), 0x00020000);
  o.ld2 = static_cast<uint32_t>(ld) * 2u;
  return o;
}

// A masked-off load is sent past the buffer's end (offsets stay below 2^31
// for valid elements), where the hardware range check returns zero.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ uint4 load16(const Operand& o, uint32_t off, bool ok) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(o.rsrc, ok ? off : kOutOfRange, 0, 0));
}

template <int R, bool KMAJ, int T>
struct Loader;

// K-contiguous rows go straight from memory into LDS (buffer_load ... lds):
// one wave instruction fills 64 consecutive 16-byte LDS chunks, i.e. 8 rows;
// lane l takes the global chunk whose swizzled position is l, so each row is
// still read as one contiguous 128-byte segment. No registers, no LDS write
// instructions; completion is waited for with vmcnt before the barrier.
template <int R, int T>
struct Loader<R, true, T> {
  static constexpr int kPerWave = R * 8 / 64 / (T / 64);  // wave instructions per tile and wave
  static_assert(kPerWave >= 1 && R * 8 % T == 0, "tile rows vs threads");

  // all of this wave's load instructions for the tile at (r0, k0); k >= kmax
  // reads zero; kofs (hi/lo segments) shifts the columns read, not the mask
  __device__ __forceinline__ void load(const Operand& o, uint4* stage, int r0, int rmax, int k0, int kmax,
                                       int kofs = 0) {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) one(o, stage, r0, rmax, k0, kmax, i, kofs);
  }
  // load instruction i of this wave
  __device__ __forceinline__ void one(const Operand& o, uint4* stage, int r0, int, int k0, int kmax, int i,
                                      int kofs = 0) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = wave * kPerWave + i;
    const int r = b * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r ^ (r >> 3)) & 7);  // global chunk stored at LDS chunk lane & 7
    const int kk = k0 + c * 8;
    const uint32_t off = static_cast<uint32_t>(r0 + r) * o.ld2 + static_cast<uint32_t>(kk + kofs) * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(o.rsrc, (__attribute__((address_space(3))) void*)(stage + b * 64),
                                             16, kk < kmax ? off : kOutOfRange, 0, 0, 0);
  }
};

// MN-contiguous operands also go straight into LDS, kept as stored: a tile
// is [64 k-rows][R] bf16, the 32-byte segment s of k-row r placed at
// segment s ^ h(r), h(r) = {0, 2, 5, 7}[r & 3]. The MFMA fragments (8
// consecutive k of one tile row) come back through the LDS transpose read
// (ds_read_b64_tr_b16): in each group of 16 lanes, lane 4 j + q addresses
// k-row j, columns 4 q .. 4 q + 3, and lane i receives column i of the 4
// k-rows. With this h the 16 lanes of a group hit distinct banks, and so do
// the 32 lanes of two neighbouring groups (4 k-rows x 2 segments).
__device__ __forceinline__ int tr_swz(int kr) { return ((kr & 3) << 1) | ((kr >> 1) & 1); }
template <int R, int T>
struct Loader<R, false, T> {
  static constexpr int kChunksRow = R / 8;                    // 16-byte chunks per k-row
  static constexpr int kPerWave = 64 * kChunksRow / 64 / (T / 64);
  static_assert(kPerWave >= 1 && kChunksRow * 64 % T == 0, "tile rows vs threads");

  __device__ __forceinline__ void load(const Operand& o, uint4* stage, int r0, int rmax, int k0, int kmax,
                                       int = 0) {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) one(o, stage, r0, rmax, k0, kmax, i);
  }
  __device__ __forceinline__ void one(const Operand& o, uint4* stage, int r0, int rmax, int k0, int kmax, int i,
                                      int = 0) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = wave * kPerWave + i;
    const int chunk = b * 64 + lane;
    const int kr = chunk / kChunksRow, cpos = chunk % kChunksRow;
    const int m = (((cpos >> 1) ^ tr_swz(kr)) << 4) + ((cpos & 1) << 3);  // tile column stored at this chunk
    const uint32_t off = static_cast<uint32_t>(k0 + kr) * o.ld2 + static_cast<uint32_t>(r0 + m) * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(o.rsrc, (__attribute__((address_space(3))) void*)(stage + b * 64),
                                             16, (r0 + m < rmax && k0 + kr < kmax) ? off : kOutOfRange, 0, 0, 0);
  }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

// The lane's MFMA fragment of tile row `row` (K-contiguous) or of the 32-row
// block starting at `row` (MN-contiguous), k-step s (16 k).
template <int R, bool KMAJ>
__device__ __forceinline__ bf16x8 read_frag(const uint4* tile, int row, int s, int lane) {
  if constexpr (KMAJ) {
    const int r = row + (lane & 31);
    return __builtin_bit_cast(bf16x8, tile[r * 8 + swz(r, 2 * s + (lane >> 5))]);
  } else {
    const int g = lane >> 4, j = (lane >> 2) & 3, q = lane & 3;
    const int kr = 16 * s + 8 * (g >> 1) + j;              // first k-row; the second read is 4 rows on
    const int mc = row + 16 * (g & 1) + 4 * q;
    const int pos = (((mc >> 4) ^ tr_swz(kr)) << 5) + ((mc & 15) << 1);
    const char* base = reinterpret_cast<const char*>(tile) + kr * (R * 2) + pos;
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 4 * R * 2));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

// EPI_SR (internal; MG_GEMM_STOCHASTIC): C = acc rounded stochastically to bf16 (a gradient).
enum Epi { EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_GELU = 2, EPI_GELU_GRAD = 3, EPI_SR = 4 };

__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Map the linear workgroup index to a tile. Workgroups are dispatched round
// robin over the 8 XCDs (each with its own L2); remap so each XCD gets a
// contiguous range, then walk that range in groups of 8 tile rows so the
// workgroups sharing an A row band or a B column band sit on one XCD.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nt = tiles_m * tiles_n;
  if ((nt & 7) == 0) pid = (pid & 7) * (nt >> 3) + (pid >> 3);
  constexpr int GM = 8;
  const int per_group = GM * tiles_n;
  const int group = pid / per_group;
  const int first = group * GM;
  const int gsize = min(tiles_m - first, GM);
  const int in_group = pid - group * per_group;
  tm = first + in_group % gsize;
  tn = in_group / gsize;
}

// Tile and split of a workgroup of a K-split product launched as a 1-D grid
// of T tiles x S splits. Workgroups go round robin over the 8 XCDs (each with
// its own L2), so workgroup L runs on XCD L % 8. The linear order here puts
// consecutive (split, tile) pairs on one XCD: the workgroups of an XCD share
// one split's K range (and so its operand k-slices, in L2), instead of the
// same few tiles over every split. Within a split, tiles go in groups of 8
// tile rows (as tile_of). Needs T * S % 8 == 0.
__device__ __forceinline__ void split_tile_of(int L, int tiles_m, int tiles_n, int S, int& tm, int& tn, int& split) {
  const int T = tiles_m * tiles_n;
  const int g = (L & 7) * (T * S >> 3) + (L >> 3);
  split = g / T;
  const int pid = g - split * T;
  constexpr int GM = 8;
  const int per_group = GM * tiles_n;
  const int group = pid / per_group;
  const int first = group * GM;
  const int gsize = min(tiles_m - first, GM);
  const int in_group = pid - group * per_group;
  tm = first + in_group % gsize;
  tn = in_group / gsize;
}

// The MFMA main loop of one workgroup tile BM x BN over k-tiles [kt0, kt1):
// WM x WN waves each accumulate (BM/WM) x (BN/WN) as 32 x 32 blocks, one
// barrier per k-tile.
// EARLY: the loads of tile t+1 are issued at the start of tile t, the
//   fragments of k-step s+1 are read under the MFMAs of step s, and the
//   barrier comes before the MFMAs of the tile's last k-step; after it tile
//   t+1 is visible to every wave, so its first fragments are read under those
//   MFMAs (faster for 256 x 256 tiles).
// otherwise: all of tile t's fragments are read, then tile t+1's loads are
//   issued, then the MFMAs run; the barrier ends the tile (the 128 x 128
//   weight-gradient tiles, two per CU).
// Either way every wave is done reading stage t & 1 at the barrier, and the
// next iteration's loads refill it.
template <int BM, int BN, int WM, int WN, bool AK, bool BKM, bool EARLY, bool INTERLEAVE = false>
__device__ __forceinline__ void mainloop(const Params& p, uint4* smem, uint4* s1, int m0, int n0, int kt0,
                                         int kt1, f32x16 (&acc)[BM / WM / 32][BN / WN / 32]) {
  constexpr int T = 64 * WM * WN;
  constexpr int MB = BM / WM / 32, NB = BN / WN / 32;  // 32x32 blocks per wave
  constexpr int S = BK / 16;                            // k-steps per tile
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const Operand oa = make_operand(p.A, p.lda, p.a_span);
  const Operand ob = make_operand(p.B, p.ldb, p.b_span);
  Loader<BM, AK, T> la;
  Loader<BN, BKM, T> lb;
  // Loads of k-tile t (relative to kt0) into stage t & 1. Past kt1 they are
  // still issued (every wave waits on the same counts) but read as zero.
  auto issue_to = [&](int t, uint4* st) {
    const KTile kt = ktile(p, kt0 + t, kt1);
    la.load(oa, st, m0, p.M, kt.k0, kt.kmax, kt.aofs);
    lb.load(ob, st + BM * 8, n0, p.N, kt.k0, kt.kmax, kt.bofs);
  };
  auto issue = [&](int t) { issue_to(t, (t & 1) ? s1 : smem); };
  const int n = kt1 - kt0;
  issue(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  int arow[MB], brow[NB];
#pragma unroll
  for (int i = 0; i < MB; ++i) arow[i] = wm * (BM / WM) + i * 32;
#pragma unroll
  for (int j = 0; j < NB; ++j) brow[j] = wn * (BN / WN) + j * 32;

  if constexpr (EARLY) {
    bf16x8 af[2][MB], bfr[2][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i) af[0][i] = read_frag<BM, AK>(smem, arow[i], 0, lane);
#pragma unroll
    for (int j = 0; j < NB; ++j) bfr[0][j] = read_frag<BN, BKM>(smem + BM * 8, brow[j], 0, lane);
    for (int t = 0; t < n; ++t) {
      issue(t + 1);
      const uint4* As = (t & 1) ? s1 : smem;
      const uint4* Bs = As + BM * 8;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int cur = s & 1;
        if (s + 1 < S) {
#pragma unroll
          for (int i = 0; i < MB; ++i) af[cur ^ 1][i] = read_frag<BM, AK>(As, arow[i], s + 1, lane);
#pragma unroll
          for (int j = 0; j < NB; ++j) bfr[cur ^ 1][j] = read_frag<BN, BKM>(Bs, brow[j], s + 1, lane);
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __syncthreads();
          if (t + 1 < n) {
            const uint4* An = ((t + 1) & 1) ? s1 : smem;
            const uint4* Bn = An + BM * 8;
#pragma unroll
            for (int i = 0; i < MB; ++i) af[cur ^ 1][i] = read_frag<BM, AK>(An, arow[i], 0, lane);
#pragma unroll
            for (int j = 0; j < NB; ++j) bfr[cur ^ 1][j] = read_frag<BN, BKM>(Bn, brow[j], 0, lane);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[cur][j], af[cur][i], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else if constexpr (INTERLEAVE) {
    // stages smem and s1 are distinct __shared__ objects, run in pairs so
    // that each is static: the reads of one then do not wait for the loads
    // into the other, and the next tile's loads are issued first
    bf16x8 af[2][MB], bfr[2][NB];
    auto tile = [&](int t, const uint4* cur, uint4* nxt) __attribute__((always_inline)) {
      issue_to(t + 1, nxt);
      const uint4* Bs = cur + BM * 8;
#pragma unroll
      for (int i = 0; i < MB; ++i) af[0][i] = read_frag<BM, AK>(cur, arow[i], 0, lane);
#pragma unroll
      for (int j = 0; j < NB; ++j) bfr[0][j] = read_frag<BN, BKM>(Bs, brow[j], 0, lane);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int c = s & 1;
        if (s + 1 < S) {
#pragma unroll
          for (int i = 0; i < MB; ++i) af[c ^ 1][i] = read_frag<BM, AK>(cur, arow[i], s + 1, lane);
#pragma unroll
          for (int j = 0; j < NB; ++j) bfr[c ^ 1][j] = read_frag<BN, BKM>(Bs, brow[j], s + 1, lane);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[c][j], af[c][i], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    };
    int t = 0;
    for (; t + 1 < n; t += 2) {
      tile(t, smem, s1);
      tile(t + 1, s1, smem);
    }
    if (t < n) tile(t, smem, s1);
  } else {
    // Every fragment of tile t is read before tile t+1's loads are issued:
    // the loads write LDS, and a read that follows them in program order
    // waits for them (the compiler cannot tell the two stages apart), which
    // would serialise each tile behind the next tile's loads. Read first, the
    // loads then fly under all of tile t's MFMAs.
    for (int t = 0; t < n; ++t) {
      const uint4* As = (t & 1) ? s1 : smem;
      const uint4* Bs = As + BM * 8;
      bf16x8 af[S][MB], bfr[S][NB];
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int i = 0; i < MB; ++i) af[s][i] = read_frag<BM, AK>(As, arow[i], s, lane);
#pragma unroll
        for (int j = 0; j < NB; ++j) bfr[s][j] = read_frag<BN, BKM>(Bs, brow[j], s, lane);
      }
      issue(t + 1);
      // keep the MFMAs between the issue and the wait (the scheduler would
      // otherwise move them past the barrier, leaving the loads no time)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[s][j], af[s][i], acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
  }
  // the zero-reading loads issued for tile n may still be landing in LDS,
  // which the epilogue reuses
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// Four-wave main loop for 256 x 256 tiles, any operand layouts: waves in
// 2 x 2, each 128 x 128 as 4 x 4 MFMA blocks, accumulators in AGPRs, one wave
// per SIMD. With one wave per SIMD nothing hides a stall of the wave's own
// instruction stream, so the k-tile is software-pipelined by hand:
//   * the two LDS stages are distinct __shared__ objects and the k-loop runs
//     tiles in pairs, so each stage is static (an LDS read is then not made
//     to wait for loads into the other stage);
//   * the next tile's loads (8 instructions per operand and wave) are spread
//     over the MFMAs of the tile's first two k-steps (A, then B: a burst
//     stalls the MFMA stream), and waited for before the last k-step;
//   * the next k-step's fragment reads are spread over the current k-step's
//     MFMAs; at the last k-step, after the tile's barrier, they are the next
//     tile's first fragments;
//   * load addresses are per-lane offsets computed once, a k-tile adds one
//     scalar; fragment addresses are computed once, k-steps are immediates.
// No load is masked: K-contiguous operands need K % 64 == 0, MN-contiguous
// ones a row count (M or N) that is a multiple of 256 (their k-rows past K lie
// past the end of the buffer and read as zero), and the prefetch after a
// split's last tile reloads that tile.

// Scheduler hints for one k-step: ND fragment reads spread over the first
// MFMAs (MD of them; early, so each read has many MFMAs to land before the
// next k-step needs it) and NV loads over the last ones.
#ifndef MG_W4_READ_SPAN
#define MG_W4_READ_SPAN 8
#endif
template <int NM, int ND, int NV, int m = 0>
__device__ __forceinline__ void interleave() {
  if constexpr (m < NM) {
    constexpr int MD = ND > MG_W4_READ_SPAN ? NM : MG_W4_READ_SPAN;  // MFMAs carrying reads
    constexpr int MV = NM / 2;                                          // MFMAs carrying loads (the last)
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    constexpr int d = m < MD ? (m + 1) * ND / MD - m * ND / MD : 0;
    constexpr int mv = m - (NM - MV);
    constexpr int v = mv >= 0 ? (mv + 1) * NV / MV - mv * NV / MV : 0;
    if constexpr (d > 0) __builtin_amdgcn_sched_group_barrier(0x100, d, 0);  // DS read
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, 0);  // VMEM read
    interleave<NM, ND, NV, m + 1>();
  }
}

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
constexpr int kW4Rows = 256;                         // tile rows per operand
constexpr int kW4Loads = kW4Rows * 8 / 64 / 4;       // load instructions per operand and wave (8)

// init<NL> / load<NL>: NL load instructions per operand and wave (the tile's
// 2048 16-byte chunks over the workgroup's waves: 8 for four waves, 4 for eight).
template <bool KMAJ>
struct W4Operand;

// K-contiguous operand: tiles [256 rows][64 k] (Loader<256, true, 256>), one
// 16-byte read per fragment.
template <>
struct W4Operand<true> {
  static constexpr int kReadsPerBlock = 1;  // fragment reads per 32-row block and k-step
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t v[kW4Loads];
  uint32_t p0, p1;  // fragment addresses of even / odd 32-row blocks
  // r0: first matrix row of the tile; wr: first tile row of this wave's 128
  template <int NL = kW4Loads>
  __device__ __forceinline__ void init(const Operand& o, int r0, int wr, int wave, int lane) {
    rsrc = o.rsrc;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int r = (wave * NL + i) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
      v[i] = static_cast<uint32_t>(r0 + r) * o.ld2 + static_cast<uint32_t>(c) * 16u;
    }
    // row wr + 32 i + L, chunk (2 s + half) ^ f(row), f(r) = (r ^ (r >> 3)) & 7;
    // f(wr + 32 i + L) = f(wr + L) ^ 4 (i & 1) for wr a multiple of 64
    const int L = lane & 31, half = lane >> 5, r = wr + L;
    p0 = static_cast<uint32_t>(r * 128 + ((half ^ ((r ^ (r >> 3)) & 7)) << 4));
    p1 = p0 ^ 64u;
  }
  __device__ __forceinline__ uint32_t koff(int k0, int kofs, uint32_t) const {
    return static_cast<uint32_t>(k0 + kofs) * 2u;
  }
  template <int NL = kW4Loads>
  __device__ __forceinline__ void load(uint4* st, int wave, int i, uint32_t ko) const {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(st + (wave * NL + i) * 64),
                                             16, v[i] + ko, 0, 0, 0);
  }
  __device__ __forceinline__ bf16x8 frag(const uint4* st, int s, int i) const {
    const uint32_t a = (((i & 1) ? p1 : p0) ^ (32u * s)) + 4096u * i;
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(st) + a));
  }
};

// MN-contiguous operand: tiles [64 k-rows][256] (Loader<256, false, 256>),
// fragments through the LDS transpose read (two 8-byte reads each).
template <>
struct W4Operand<false> {
  static constexpr int kReadsPerBlock = 2;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t v[kW4Loads];
  uint32_t fb[4];  // byte address of block i's first read at k-step 0
  template <int NL = kW4Loads>
  __device__ __forceinline__ void init(const Operand& o, int r0, int wr, int wave, int lane) {
    rsrc = o.rsrc;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int chunk = (wave * NL + i) * 64 + lane;
      const int kr = chunk >> 5, cpos = chunk & 31;
      const int m = (((cpos >> 1) ^ tr_swz(kr)) << 4) + ((cpos & 1) << 3);
      v[i] = static_cast<uint32_t>(kr) * o.ld2 + static_cast<uint32_t>(r0 + m) * 2u;
    }
    // read_frag<256, false>: k-row 16 s + 8 (g >> 1) + j, column wr + 32 i + 16 (g & 1) + 4 q;
    // tr_swz of that k-row is tr_swz(j) (the xor is applied to the absolute
    // 16-column block index, which the loader swizzled the same way)
    const int g = lane >> 4, j = (lane >> 2) & 3, q = lane & 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int colblk = (wr >> 4) + 2 * i + (g & 1);
      fb[i] = static_cast<uint32_t>((8 * (g >> 1) + j) * (kW4Rows * 2) + ((colblk ^ tr_swz(j)) << 5) + 8 * q);
    }
  }
  __device__ __forceinline__ uint32_t koff(int k0, int, uint32_t ld2) const { return static_cast<uint32_t>(k0) * ld2; }
  template <int NL = kW4Loads>
  __device__ __forceinline__ void load(uint4* st, int wave, int i, uint32_t ko) const {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(st + (wave * NL + i) * 64),
                                             16, v[i] + ko, 0, 0, 0);
  }
  __device__ __forceinline__ bf16x8 frag(const uint4* st, int s, int i) const {
    const char* base = reinterpret_cast<const char*>(st) + fb[i] + 16 * s * (kW4Rows * 2);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 4 * kW4Rows * 2));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

template <bool AK, bool BKM>
__device__ __forceinline__ void mainloop_w4(const Params& p, uint4* sa, uint4* sb, int m0, int n0, int kt0, int kt1,
                                            f32x16 (&acc)[4][4]) {
  constexpr int S = BK / 16;
  constexpr int kStageA = kW4Rows * 8;  // uint4 of the A tile (B follows)
  // the wave index in a scalar register: the loads' LDS destinations (M0) are then scalar arithmetic
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  const Operand oa = make_operand(p.A, p.lda, p.a_span);
  const Operand ob = make_operand(p.B, p.ldb, p.b_span);
  W4Operand<AK> A;
  W4Operand<BKM> B;
  A.init(oa, m0, wm * 128, wave, lane);
  B.init(ob, n0, wn * 128, wave, lane);
  // byte offsets of k-tile t (relative to kt0); tiles past kt1 reload tile kt1 - 1
  auto koffs = [&](int t, uint32_t& ao, uint32_t& bo) {
    const int tg = min(kt0 + t, kt1 - 1);
    int seg = 0, k0 = tg * BK;
    if (p.hilo) {  // K-contiguous only (checked by the host)
      seg = tg / p.nkt_seg;
      k0 = (tg - seg * p.nkt_seg) * BK;
    }
    ao = A.koff(k0, seg == 1 ? p.K : 0, oa.ld2);
    bo = B.koff(k0, seg == 2 ? p.K : 0, ob.ld2);
  };
  bf16x8 af[2][4], bfr[2][4];
  // in the order the MFMAs need them: (i, j) loops i outer, so A_0 and all of B first
  auto read_step = [&](const uint4* st, int s, int buf) {
    af[buf][0] = A.frag(st, s, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[buf][j] = B.frag(st + kStageA, s, j);
#pragma unroll
    for (int i = 1; i < 4; ++i) af[buf][i] = A.frag(st, s, i);
  };
  auto mfma_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[buf][j], af[buf][i], acc[i][j], 0, 0, 0);
  };
  constexpr int NR = 4 * (W4Operand<AK>::kReadsPerBlock + W4Operand<BKM>::kReadsPerBlock);  // reads per k-step
  const int n = kt1 - kt0;
  {
    uint32_t ao, bo;
    koffs(0, ao, bo);
#pragma unroll
    for (int i = 0; i < kW4Loads; ++i) A.load(sa, wave, i, ao);
#pragma unroll
    for (int i = 0; i < kW4Loads; ++i) B.load(sa + kStageA, wave, i, bo);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  read_step(sa, 0, 0);
  // one k-tile from `cur`, loading tile t + 1 into `nxt`
  auto tile = [&](int t, const uint4* cur, uint4* nxt) __attribute__((always_inline)) {
    uint32_t ao, bo;
    koffs(t + 1, ao, bo);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int c = s & 1;
      if (s == 0) {
#pragma unroll
        for (int i = 0; i < kW4Loads; ++i) A.load(nxt, wave, i, ao);
      } else if (s == 1) {
#pragma unroll
        for (int i = 0; i < kW4Loads; ++i) B.load(nxt + kStageA, wave, i, bo);
      }
      if (s + 1 < S) {
        read_step(cur, s + 1, c ^ 1);
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // tile t + 1 is in `nxt` for every wave; every wave is done with `cur`
        read_step(nxt, 0, c ^ 1);
      }
      mfma_step(c);
      if (s < 2) interleave<16, NR, kW4Loads>();
      else interleave<16, NR, 0>();
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int t = 0;
  for (; t + 1 < n; t += 2) {
    tile(t, sa, sb);
    tile(t + 1, sb, sa);
  }
  if (t < n) tile(t, sa, sb);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// Eight-wave pipelined main loop, 256 x 256 tiles: mainloop_w4's stage
// pipeline with two waves per SIMD, each owning 64 x 128 of the tile (2 x 4
// blocks, 128 accumulator registers), all eight multiplying at once. A second
// wave per SIMD keeps the matrix core busier than one wave issuing back to
// back (measured on random operands: about 1.8-2.0 against 1.7 PFLOP/s for
// 32x32x16 bf16), at 1.5x the fragment reads per MFMA of the 128 x 128 wave
// tile. Waves 0-3 (one per SIMD) also issue the tile loads, 16 per k-tile
// each, so every SIMD has one wave whose MFMA stream no load interrupts
// (measured 4-6% faster than all eight waves loading).
template <bool AK, bool BKM>
__device__ __forceinline__ void mainloop_w8(const Params& p, uint4* sa, uint4* sb, int m0, int n0, int kt0, int kt1,
                                            f32x16 (&acc)[2][4]) {
  constexpr int S = BK / 16;
  constexpr int kLoaders = 4;                  // waves 0..3 load
  constexpr int NL = kW4Loads * 4 / kLoaders;  // load instructions per operand and loading wave
  constexpr int kStageA = kW4Rows * 8;         // uint4 of the A tile (B follows)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // tile rows 64 wm .., columns 128 wn ..
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  const Operand oa = make_operand(p.A, p.lda, p.a_span);
  const Operand ob = make_operand(p.B, p.ldb, p.b_span);
  W4Operand<AK> A;
  W4Operand<BKM> B;
  A.template init<NL>(oa, m0, wm * 64, wave % kLoaders, lane);
  B.template init<NL>(ob, n0, wn * 128, wave % kLoaders, lane);
  auto koffs = [&](int t, uint32_t& ao, uint32_t& bo) {
    const int tg = min(kt0 + t, kt1 - 1);
    int seg = 0, k0 = tg * BK;
    if (p.hilo) {
      seg = tg / p.nkt_seg;
      k0 = (tg - seg * p.nkt_seg) * BK;
    }
    ao = A.koff(k0, seg == 1 ? p.K : 0, oa.ld2);
    bo = B.koff(k0, seg == 2 ? p.K : 0, ob.ld2);
  };
  bf16x8 af[2][2], bfr[2][4];
  auto read_step = [&](const uint4* st, int s, int buf) {
    af[buf][0] = A.frag(st, s, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[buf][j] = B.frag(st + kStageA, s, j);
    af[buf][1] = A.frag(st, s, 1);
  };
  auto mfma_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[buf][j], af[buf][i], acc[i][j], 0, 0, 0);
  };
  constexpr int NR = 2 * W4Operand<AK>::kReadsPerBlock + 4 * W4Operand<BKM>::kReadsPerBlock;
  const int n = kt1 - kt0;
  // The whole loop once per role, so a loading wave's loads and MFMAs share
  // one instruction block (and one schedule).
  auto run = [&](auto role) __attribute__((always_inline)) {
    constexpr bool kLoad = decltype(role)::value;
    if constexpr (kLoad) {
      uint32_t ao, bo;
      koffs(0, ao, bo);
#pragma unroll
      for (int i = 0; i < NL; ++i) A.template load<NL>(sa, wave, i, ao);
#pragma unroll
      for (int i = 0; i < NL; ++i) B.template load<NL>(sa + kStageA, wave, i, bo);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    read_step(sa, 0, 0);
    auto tile = [&](int t, const uint4* cur, uint4* nxt) __attribute__((always_inline)) {
      uint32_t ao = 0, bo = 0;
      if constexpr (kLoad) koffs(t + 1, ao, bo);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int c = s & 1;
        if constexpr (kLoad) {
          if (s == 0) {
#pragma unroll
            for (int i = 0; i < NL; ++i) A.template load<NL>(nxt, wave, i, ao);
          } else if (s == 1) {
#pragma unroll
            for (int i = 0; i < NL; ++i) B.template load<NL>(nxt + kStageA, wave, i, bo);
          }
        }
        if (s + 1 < S) {
          read_step(cur, s + 1, c ^ 1);
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __syncthreads();  // tile t + 1 is in `nxt` for every wave; every wave is done with `cur`
          read_step(nxt, 0, c ^ 1);
        }
        mfma_step(c);
        if (kLoad && s < 2) interleave<8, NR, NL>();
        else interleave<8, NR, 0>();
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    int t = 0;
    for (; t + 1 < n; t += 2) {
      tile(t, sa, sb);
      tile(t + 1, sb, sa);
    }
    if (t < n) tile(t, sa, sb);
  };
  if (wave < kLoaders) run(std::true_type{});
  else run(std::false_type{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// ---------------------------------------------------------------- 16x16x32 four-wave loop
#ifndef MG_GEMM_W4M
#define MG_GEMM_W4M 1
#endif
constexpr bool kUseW4M = MG_GEMM_W4M != 0;

//
// mainloop_w4m: 256 x 256 tiles, four waves (one per SIMD) of 128 x 128, each
// as 8 x 8 blocks of v_mfma_f32_16x16x32_bf16 (f32x4 accumulators, 256
// registers a lane, in AGPRs). Measured on MI355X with random operands, the
// 16x16x32 instruction draws less energy per flop than 32x32x16 (register-only
// microbenchmark: 2.02 against 1.75-1.79 PFLOP/s, at 2.04-2.09 against
// 1.75-1.78 GHz), and these products are power-bound; a 128 x 128 wave tile
// reads half the LDS fragment bytes per flop of a 64 x 128 one.
// A k-tile (64 k) is two k-steps of 32:
//   k-step 0: 64 MFMAs on fragments of k-step 0; k-step 1's fragments read
//             under them;
//   mid-tile: wait for this wave's loads of tile t + 1, then the barrier:
//             tile t + 1 is in its stage for every wave, and every wave has
//             read all of tile t's fragments (so its stage is free);
//   k-step 1: 64 MFMAs; under them the loads of tile t + 2 into tile t's
//             stage and the reads of tile t + 1's k-step 0 fragments.
// Loads therefore have a k-tile and a half of MFMAs to land (the loop before
// this one gave them two k-steps of 16).
// LDS layouts (both distinct from the other loops'):
//   K-contiguous: [256 rows][8 chunks of 16 B], chunk c of row r at
//     c ^ f(r), f(r) = (r & 7) ^ ((r >> 3) & 1). A fragment (16 rows, 8 k
//     each for the four 16-lane groups) is one 16-byte read per lane; the 16
//     rows of a lane group land in 16 distinct 16-byte bank groups.
//   MN-contiguous: [64 k-rows][256], the 32-byte segment s of k-row r at
//     s ^ t16(r), t16(r) = tr_swz(r) ^ (((r >> 3) & 1) << 2); fragments come
//     through two LDS transpose reads (4 k-rows each).
// Loads: every wave issues 8 per operand and k-tile.
// Load placement in a k-step (A/B'd on MI355X at the cfg3 shapes: one load
// every three MFMAs from MFMA 1 beat groups of 2 and 4 and a burst by 1-10%)
#ifndef MG_W4M_LOAD_FIRST
#define MG_W4M_LOAD_FIRST 1
#endif
#ifndef MG_W4M_LOAD_EVERY
#define MG_W4M_LOAD_EVERY 3
#endif
#ifndef MG_W4M_LOAD_GROUP
#define MG_W4M_LOAD_GROUP 1
#endif
__device__ __forceinline__ int tr_swz16(int kr) { return tr_swz(kr) ^ (((kr >> 3) & 1) << 2); }

template <bool KMAJ>
struct M16Operand;

// Offsets of the loads: everything that decides whether an element lies
// inside the operand (the row for a K-contiguous operand, the k-row for an
// MN-contiguous one) is in the per-lane (VGPR) offset, which the buffer's
// range check covers, so rows past M and k-rows past K read as zero; only
// offsets that stay inside the operand for every in-range element (the
// k-tile's columns of a K-contiguous operand, the tile's first column of an
// MN-contiguous one, whose row count is a multiple of 256) go into the scalar
// offset. The per-lane offsets are relative to the tile origin; load() adds
// the origin (a scalar per tile, so a persistent kernel can load the next
// tile's k-tiles).
template <>
struct M16Operand<true> {
  static constexpr int kReads = 1;  // LDS reads per fragment
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t v[8];  // load i: byte offset of the lane's row and chunk within the tile
  uint32_t q[2];  // byte address of block 0's fragment at k-step s
  // wr: first tile row of this wave's 128
  __device__ __forceinline__ void init(const Operand& o, int wr, int wave, int lane) {
    rsrc = o.rsrc;
    // load i of wave w fills rows (8 w + i) 8 + (lane >> 3), whose f is
    // (lane >> 3) ^ (i & 1); lane l's LDS chunk l & 7 takes global chunk (l & 7) ^ f
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = static_cast<uint32_t>(wave * 64 + i * 8 + (lane >> 3)) * o.ld2 +
             static_cast<uint32_t>(((lane & 7) ^ (lane >> 3) ^ (i & 1)) << 4);
    // fragment: lane l reads row wr + 16 I + (l & 15), chunk 4 s + (l >> 4);
    // f of that row does not depend on I
    const int hl = lane >> 4, r = wr + (lane & 15);
    const int f = (r & 7) ^ ((r >> 3) & 1);
#pragma unroll
    for (int s = 0; s < 2; ++s) q[s] = static_cast<uint32_t>(r * 128 + ((((4 * s) | hl) ^ f) << 4));
  }
  // byte offset of a tile whose first row is r0
  __device__ __forceinline__ static uint32_t origin(int r0, uint32_t ld2) { return static_cast<uint32_t>(r0) * ld2; }
  // the k-tile's offset (scalar): k0 (+ kofs, the hi/lo segment) columns
  __device__ __forceinline__ uint32_t koff(int k0, int kofs, uint32_t) const {
    return static_cast<uint32_t>(k0 + kofs) * 2u;
  }
  __device__ __forceinline__ void load(uint4* st, int wave, int i, uint32_t ko, uint32_t org) const {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(st + (wave * 8 + i) * 64),
                                             16, v[i] + org, ko, 0, 0);
  }
  __device__ __forceinline__ bf16x8 frag(const uint4* st, int s, int I) const {
    const uint32_t a = q[s] + 2048u * I;
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(st) + a));
  }
  // Hides the fragment base addresses from loop-invariant hoisting, so each
  // read is base + immediate (else one register per fragment address).
  __device__ __forceinline__ void opaque() { asm volatile("" : "+v"(q[0]), "+v"(q[1])); }
};

template <>
struct M16Operand<false> {
  static constexpr int kReads = 2;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t v[8];  // load i: k-row (of the k-tile) and column (of the tile) of the lane, in bytes
  uint32_t z;     // byte address of the lane's first transpose read (block 0, k-step 0)
  __device__ __forceinline__ void init(const Operand& o, int wr, int wave, int lane) {
    rsrc = o.rsrc;
    // load i of wave w fills k-row (8 w + i) 2 + h (h = lane >> 5), chunk
    // c = lane & 31 of it: tile column 16 ((c >> 1) ^ t16(k-row)) + 8 (c & 1)
    const int h = lane >> 5, cpos = lane & 31;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kr = (wave * 8 + i) * 2 + h;
      const int m = (((cpos >> 1) ^ tr_swz16(kr)) << 4) + ((cpos & 1) << 3);
      v[i] = static_cast<uint32_t>(kr) * o.ld2 + static_cast<uint32_t>(m) * 2u;
    }
    // fragment J: column wr + 16 J + (l & 15), k-rows 32 s + 8 g + 0..7
    // (g = l >> 4): in each 16-lane group lane 4 j + q addresses k-row
    // 8 g + j, columns 4 q .. 4 q + 3 of the 16-column block
    const int g = lane >> 4, j = (lane >> 2) & 3, qq = lane & 3;
    const int kr = 8 * g + j;
    z = static_cast<uint32_t>(kr * (kW4Rows * 2) + (((wr >> 4) ^ tr_swz16(kr)) << 5) + 8 * qq);
  }
  __device__ __forceinline__ static uint32_t origin(int r0, uint32_t) { return static_cast<uint32_t>(r0) * 2u; }
  // the k-tile's offset: k0 k-rows (added to the per-lane offset, which the range check covers)
  __device__ __forceinline__ uint32_t koff(int k0, int, uint32_t ld2) const { return static_cast<uint32_t>(k0) * ld2; }
  __device__ __forceinline__ void load(uint4* st, int wave, int i, uint32_t ko, uint32_t org) const {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(st + (wave * 8 + i) * 64),
                                             16, v[i] + ko, org, 0, 0);
  }
  __device__ __forceinline__ void opaque() { asm volatile("" : "+v"(z)); }
  // (wr >> 4) is a multiple of 8, so block J's segment is that of block 0 ^ J
  __device__ __forceinline__ bf16x8 frag(const uint4* st, int s, int J) const {
    const char* base =
        reinterpret_cast<const char*>(st) + (z ^ (static_cast<uint32_t>(J) << 5)) + 32 * s * (kW4Rows * 2);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 4 * kW4Rows * 2));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

// acc += B A on v_mfma_f32_16x16x32_bf16 with acc held in AGPRs and tied
// (dst = srcC). Written as inline assembly because with 64 separate
// four-register accumulators filling all 256 AGPRs the register allocator,
// given the builtin, moved accumulators between registers (hundreds of
// v_accvgpr moves per k-tile, measured in the assembly); with the operand
// pinned it keeps each in place. The compiler's hazard checks do not see
// into the assembly, so mainloop_w4m keeps every hazard away by
// construction:
//   * no VALU writes an accumulator: the first k-step uses the srcC = 0 form
//     (mfma16_agpr_first) instead of a zero fill;
//   * after the last k-step, mfma16_agpr_drain holds the epilogue's reads of
//     the accumulators written by the last 16 MFMAs behind 24 wait states
//     (more than a 16-pass XDL write needs before a VALU read); every other
//     accumulator was written 16 or more MFMAs before the end;
//   * a fragment's VGPRs are refilled from LDS at least 11 MFMAs after the
//     last MFMA that read them, and each accumulator is next read as srcC 64
//     MFMAs after it was written.
__device__ __forceinline__ void mfma16_agpr(f32x4v& acc, const bf16x8& b, const bf16x8& a) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(b), "v"(a));
}
__device__ __forceinline__ void mfma16_agpr_first(f32x4v& acc, const bf16x8& b, const bf16x8& a) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(b), "v"(a));
}
// 24 wait states after the MFMAs that wrote acc[6][*] and acc[7][*]; any read
// of them depends on this statement's outputs and so comes after it.
__device__ __forceinline__ void mfma16_agpr_drain(f32x4v (&acc)[8][8]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(acc[6][0]), "+a"(acc[6][1]), "+a"(acc[6][2]), "+a"(acc[6][3]), "+a"(acc[6][4]),
                 "+a"(acc[6][5]), "+a"(acc[6][6]), "+a"(acc[6][7]), "+a"(acc[7][0]), "+a"(acc[7][1]),
                 "+a"(acc[7][2]), "+a"(acc[7][3]), "+a"(acc[7][4]), "+a"(acc[7][5]), "+a"(acc[7][6]),
                 "+a"(acc[7][7]));
}

// ---------------------------------------------------------------- bf16 GELU by table
// bf16(gelu(x)) for a bf16 x (gelu() of mg_common.h, rounded to nearest), as a
// function of its 16 bits b, mag = b & 0x7fff:
//   2^-9 <= |x| < 2^15 (biased exponent 118 .. 141): a table of 24 exponents
//     x 128 mantissas x 2 signs (12 KB), entry 2 (mag - 0x3b00) + sign, filled
//     from gelu() itself by each workgroup;
//   2^-125 <= |x| < 2^-9: b - 0x80, i.e. x / 2. The erf term moves x / 2 by
//     less than 0.8 |x| < 2^-9.3 relatively, under half a bf16 spacing, and
//     x / 2 is itself a bf16 value;
//   anything else (zero, subnormals, |x| >= 2^15, inf, NaN) is exceptional:
//     flagged, and its chunk recomputed with gelu() (gelu_exact_chunk) under
//     a wave-uniform branch.
// So every result equals bf16(gelu(x)); a lookup is ~12 VALU operations and
// one LDS read, against ~30 for erf.
constexpr int kGeluLutN = 2 * 24 * 128;
__device__ __forceinline__ void gelu_lut_fill(uint16_t* lut) {
  for (int i = threadIdx.x; i < kGeluLutN; i += blockDim.x) {
    const uint32_t b = ((static_cast<uint32_t>(i) & 1u) << 15) | ((static_cast<uint32_t>(i) >> 1) + 0x3b00u);
    lut[i] = f32_to_bf16(gelu(__uint_as_float(b << 16)));
  }
}
// table index of a value with magnitude bits mag and sign bit sg (clamped into
// the table outside its range, where the entry is not used)
__device__ __forceinline__ uint32_t gelu_lut_index(uint32_t mag, uint32_t sg) {
  const int d = min(max(static_cast<int>(mag) - 0x3b00, 0), kGeluLutN / 2 - 1);
  return static_cast<uint32_t>(d) * 2u + sg;
}
// is a value exceptional (outside both the table and the x / 2 range)?
__device__ __forceinline__ bool gelu_exceptional(uint32_t mag) { return mag - 0x100u > 0x45ffu; }
// bf16(gelu) of 8 bf16 values (one 16-byte chunk) from the table; exc is set
// if one of them is exceptional (the result is then not used). The 8 table
// reads are issued together (one LDS round trip per chunk).
__device__ __forceinline__ uint4 gelu_lut_chunk(const uint4& w, const uint16_t* lut, bool& exc) {
  const uint32_t wi[4] = {w.x, w.y, w.z, w.w};
  uint32_t b[8], t[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) b[v] = (v & 1) ? (wi[v >> 1] >> 16) : (wi[v >> 1] & 0xffffu);
#pragma unroll
  for (int v = 0; v < 8; ++v) t[v] = lut[gelu_lut_index(b[v] & 0x7fffu, b[v] >> 15)];
  uint32_t wo[4] = {0, 0, 0, 0};
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const uint32_t mag = b[v] & 0x7fffu;
    exc = exc || gelu_exceptional(mag);
    const uint32_t y = mag < 0x3b00u ? b[v] - 0x80u : t[v];
    wo[v >> 1] |= (v & 1) ? (y << 16) : y;
  }
  return make_uint4(wo[0], wo[1], wo[2], wo[3]);
}
// bf16(gelu) of 8 bf16 values (one 16-byte chunk) by gelu() itself
__device__ __forceinline__ uint4 gelu_exact_chunk(const uint4& w) {
  const uint32_t wi[4] = {w.x, w.y, w.z, w.w};
  uint32_t wo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    wo[e] = pack_bf16x2(gelu(__uint_as_float(wi[e] << 16)), gelu(__uint_as_float(wi[e] & 0xffff0000u)));
  return make_uint4(wo[0], wo[1], wo[2], wo[3]);
}

// The pre-activation (aux) of the bias + GELU epilogue: a non-temporal store.
// It is read again only by the backward pass, long after; stored normally it
// takes the place in the memory-side cache of the activation written beside
// it, which the next product reads at once (that product measured ~10% slower
// with the activation half evicted).
__device__ __forceinline__ void store_aux(bf16_t* dst, const uint4& v) {
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(dst));
}

// f(std::integral_constant<int, M>{}) for each M, in order (a loop whose index
// is a compile-time constant in the body)
template <int... M, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, M...>, F&& f) {
  (f(std::integral_constant<int, M>{}), ...);
}

// The four-wave 16x16x32 pipeline's per-wave state (operand offsets, fragment
// buffers) and its steps, shared by mainloop_w4m and gemm_persist_w4m_kernel.
template <bool AK, bool BKM>
struct W4MPipe {
  static constexpr int kStageA = kW4Rows * 8;  // uint4 of the A tile (B follows)
  static constexpr int NR = 8 * (M16Operand<AK>::kReads + M16Operand<BKM>::kReads);  // LDS reads per k-step
  Operand oa, ob;
  M16Operand<AK> A;
  M16Operand<BKM> B;
  bf16x8 af[2][8], bfr[2][8];
  int wave, nseg, K;

  __device__ __forceinline__ void init(const Params& p, int wave_, int lane) {
    wave = wave_;
    oa = make_operand(p.A, p.lda, p.a_span);
    ob = make_operand(p.B, p.ldb, p.b_span);
    A.init(oa, (wave >> 1) * 128, wave, lane);
    B.init(ob, (wave & 1) * 128, wave, lane);
    nseg = p.hilo ? p.nkt_seg : (1 << 29);  // k-tiles per hi/lo segment (none: never reached; 2 nseg < 2^31)
    K = p.K;
  }
  // a tile of a product whose hi/lo mode varies by tile (Params::hilo_cols)
  __device__ __forceinline__ void set_hilo(const Params& p, bool hilo_tile) {
    nseg = __builtin_amdgcn_readfirstlane(hilo_tile ? p.nkt_seg : (1 << 29));  // wave-uniform: a scalar
  }
  // byte offsets of the tile origins (m0, n0)
  __device__ __forceinline__ uint32_t aorg(int m0) const { return M16Operand<AK>::origin(m0, oa.ld2); }
  __device__ __forceinline__ uint32_t borg(int n0) const { return M16Operand<BKM>::origin(n0, ob.ld2); }
  // k offsets of k-tile tg of the product. Branch-free (selects), so the
  // k-loop stays one basic block.
  __device__ __forceinline__ void koffs(int tg, uint32_t& ao, uint32_t& bo) const {
    const int seg = tg >= 2 * nseg ? 2 : (tg >= nseg ? 1 : 0);
    const int k0 = (tg - seg * nseg) * BK;
    ao = A.koff(k0, seg == 1 ? K : 0, oa.ld2);
    bo = B.koff(k0, seg == 2 ? K : 0, ob.ld2);
  }
  __device__ __forceinline__ void load_tile(uint4* st, uint32_t ao, uint32_t bo, uint32_t ar, uint32_t br) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) A.load(st, wave, i, ao, ar);
#pragma unroll
    for (int i = 0; i < 8; ++i) B.load(st + kStageA, wave, i, bo, br);
  }
  // fragment r (0..15) of a k-step, in the order the MFMAs need them (I
  // outer): A_0, B_0 .. B_7, A_1 .. A_7
  __device__ __forceinline__ void read_frag(const uint4* st, int s, int buf, int r) {
    if (r == 0)
      af[buf][0] = A.frag(st, s, 0);
    else if (r <= 8)
      bfr[buf][r - 1] = B.frag(st + kStageA, s, r - 1);
    else
      af[buf][r - 8] = A.frag(st, s, r - 8);
  }
  __device__ __forceinline__ void read_all(const uint4* st, int s, int buf) {
#pragma unroll
    for (int r = 0; r < 16; ++r) read_frag(st, s, buf, r);
  }
  __device__ __forceinline__ void opaque() {
    A.opaque();  // (volatile asm orders memory operations: before the loads)
    B.opaque();
  }
  // One k-step in a fixed instruction order (a scheduling barrier after each
  // MFMA keeps the compiler from reordering): the 64 MFMAs on fragment buffer
  // CB (kFirst: acc = product, the first k-step of a tile); after MFMA 3 r,
  // fragment r of the next k-step (stage rst, k-step rs) into buffer 1 - CB;
  // the 16 loads of a k-tile (offsets ao, bo, origins ar, br) into stage lst,
  // MG_W4M_LOAD_GROUP after MFMA MG_W4M_LOAD_FIRST + MG_W4M_LOAD_EVERY g.
  template <int CB, bool kReads, bool kLoads, bool kFirst>
  __device__ __forceinline__ void kstep(f32x4v (&acc)[8][8], const uint4* rst, int rs, uint4* lst, uint32_t ao,
                                        uint32_t bo, uint32_t ar, uint32_t br) {
    constexpr int LF = MG_W4M_LOAD_FIRST, LE = MG_W4M_LOAD_EVERY, LG = MG_W4M_LOAD_GROUP;
    static_for(std::make_integer_sequence<int, 64>{}, [&](auto mc) __attribute__((always_inline)) {
      constexpr int m = decltype(mc)::value;
      constexpr int i = m >> 3, j = m & 7;
      if constexpr (kFirst)
        mfma16_agpr_first(acc[i][j], bfr[CB][j], af[CB][i]);
      else
        mfma16_agpr(acc[i][j], bfr[CB][j], af[CB][i]);
      if constexpr (kReads) {
        if constexpr (m % 3 == 0 && m / 3 < 16) read_frag(rst, rs, 1 - CB, m / 3);
      }
      if constexpr (kLoads) {
        if constexpr (m >= LF && (m - LF) % LE == 0 && (m - LF) / LE < 16 / LG) {
#pragma unroll
          for (int v = (m - LF) / LE * LG; v < ((m - LF) / LE + 1) * LG; ++v) {
            if (v < 8)
              A.load(lst, wave, v, ao, ar);
            else
              B.load(lst + kStageA, wave, v - 8, bo, br);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  }
};

template <bool AK, bool BKM>
__device__ __forceinline__ void mainloop_w4m(const Params& p, uint4* sa, uint4* sb, int m0, int n0, int kt0, int kt1,
                                             f32x4v (&acc)[8][8]) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  W4MPipe<AK, BKM> P;
  P.init(p, wave, lane);
  const uint32_t ar = P.aorg(m0), br = P.borg(n0);
  // k offsets of k-tile t (relative to kt0); tiles past kt1 reload tile kt1 - 1
  auto koffs = [&](int t, uint32_t& ao, uint32_t& bo) { P.koffs(min(kt0 + t, kt1 - 1), ao, bo); };
  const int n = kt1 - kt0;
  // prologue: tiles 0 and 1 in flight, tile 0's k-step 0 multiplied, then the
  // mid-tile barrier of tile 0
  uint32_t ao, bo;
  koffs(0, ao, bo);
  P.load_tile(sa, ao, bo, ar, br);
  koffs(1, ao, bo);
  P.load_tile(sb, ao, bo, ar, br);
  asm volatile("s_waitcnt vmcnt(16)" ::: "memory");  // tile 0 (tile 1's 16 loads may still be in flight)
  __syncthreads();
  P.read_all(sa, 0, 0);
  P.template kstep<0, true, false, true>(acc, sa, 1, sa, 0, 0, ar, br);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // From the mid-tile barrier of tile t to that of tile t + 1. No load is in
  // flight at either end, so the loop's back edge carries none (the compiler
  // then adds no wait of its own for the direct-to-LDS writes):
  //   k-step 1 of tile t: the loads of tile t + 2 into `cur` (tile t's stage,
  //     read out by now), tile t + 1's k-step 0 fragments read from `nxt`;
  //   k-step 0 of tile t + 1, reading its k-step 1 fragments;
  //   wait for the loads, barrier.
  auto unit = [&](int t, uint4* cur, const uint4* nxt) __attribute__((always_inline)) {
    P.opaque();
    uint32_t lo, lb;
    koffs(t + 2, lo, lb);
    P.template kstep<1, true, true, false>(acc, nxt, 0, cur, lo, lb, ar, br);
    P.template kstep<0, true, false, false>(acc, nxt, 1, cur, 0, 0, ar, br);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // tile t + 2 is in `cur` for every wave; every wave is done with `nxt`
  };
  int t = 0;
  for (; t + 2 < n; t += 2) {
    unit(t, sa, sb);
    unit(t + 1, sb, sa);
  }
  if (t + 1 < n) unit(t, sa, sb);
  // k-step 1 of the last tile (its fragments are in buffer 1)
  P.template kstep<1, false, false, false>(acc, sa, 0, sa, 0, 0, ar, br);
  mfma16_agpr_drain(acc);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// Ping-pong main loop, 256 x 256 tiles, 8 waves in two groups of four (one
// wave of each group per SIMD; group g owns tile rows 128 g .. 128 g + 127,
// each wave 128 x 64). The groups alternate, a workgroup barrier between
// phases: while one group multiplies a whole k-tile from registers, the
// other reads its fragments of that k-tile from LDS.
//   phase 2t:   group 0 reads tile t        group 1 multiplies tile t-1
//   phase 2t+1: group 0 multiplies tile t   group 1 reads tile t
// Every wave issues its share of tile t+1's loads at the start of phase 2t
// (stage t+1 & 1 was last read in phase 2t-1) and waits for them at the end
// of phase 2t+1. (Spreading the loads between the reads and MFMAs measured
// slower for this operand layout.)
template <bool AK, bool BKM>
__device__ __forceinline__ void mainloop_pp(const Params& p, uint4* smem, int m0, int n0, int kt0, int kt1,
                                            f32x16 (&acc)[4][2]) {
  constexpr int BM = 256, BN = 256, T = 512, MB = 4, NB = 2, S = BK / 16;
  constexpr int kStage = (BM + BN) * 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / 4, wn = wave % 4;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  const Operand oa = make_operand(p.A, p.lda, p.a_span);
  const Operand ob = make_operand(p.B, p.ldb, p.b_span);
  Loader<BM, AK, T> la;
  Loader<BN, BKM, T> lb;
  constexpr int LA = decltype(la)::kPerWave, LB = decltype(lb)::kPerWave;
  static_assert(LA + LB == 2 * S, "two load instructions per k-step");
  const int kmax = min(p.K, kt1 * BK);  // (no hi/lo products on this loop)
  auto dma = [&](int t, int q) {  // load instruction q of k-tile t
    uint4* st = smem + ((t & 1) * kStage);
    if (q < LA) la.one(oa, st, m0, p.M, (kt0 + t) * BK, kmax, q);
    else lb.one(ob, st + BM * 8, n0, p.N, (kt0 + t) * BK, kmax, q - LA);
  };

  // K-contiguous fragment (tile row r = r0 + 32 i + lane % 32, k-step s) at
  // byte r * 128 + (((2 s + half) ^ f(r)) * 16), f(r) = (r ^ (r >> 3)) & 7.
  // f(r0 + 32 i + l) = f(r0 + l) ^ (4 if i is odd), so with
  // P_par = (r0 + l) * 128 + ((half ^ f(r0 + l) ^ 4 par) * 16) the address
  // is (P_{i&1} ^ 32 s) + 4096 i. The xor is redone at each read (volatile)
  // instead of keeping 16 addresses live next to 224 registers of
  // fragments and accumulators.
  const int L = lane & 31, half = lane >> 5;
  auto kbase = [&](int r0, int par) -> uint32_t {
    const int r = r0 + L;
    return static_cast<uint32_t>(r * 128 + (((half ^ ((r ^ (r >> 3)) & 7)) ^ (4 * par)) << 4));
  };
  const uint32_t pa0 = kbase(wm * 128, 0), pa1 = kbase(wm * 128, 1);
  const uint32_t pb0 = kbase(wn * 64, 0), pb1 = kbase(wn * 64, 1);
  auto kread = [&](const uint4* tile, uint32_t P, int s, int i) -> bf16x8 {
    uint32_t x;
    asm volatile("v_xor_b32 %0, %1, %2" : "=v"(x) : "n"(32 * s), "v"(P));
    return __builtin_bit_cast(bf16x8,
                              *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(tile) + x + 4096 * i));
  };
  bf16x8 fa[S][MB], fb[S][NB];
  auto frag_a = [&](const uint4* As, int s, int i) -> bf16x8 {
    if constexpr (AK) return kread(As, (i & 1) ? pa1 : pa0, s, i);
    else return read_frag<BM, AK>(As, wm * 128 + i * 32, s, lane);
  };
  auto frag_b = [&](const uint4* Bs, int s, int j) -> bf16x8 {
    if constexpr (BKM) return kread(Bs, (j & 1) ? pb1 : pb0, s, j);
    else return read_frag<BN, BKM>(Bs, wn * 64 + j * 32, s, lane);
  };
  auto issue = [&](int t) {
#pragma unroll
    for (int q = 0; q < LA + LB; ++q) dma(t, q);
  };
  // all fragments of tile t
  auto read_all = [&](int t) {
    const uint4* As = smem + (t & 1) * kStage;
    const uint4* Bs = As + BM * 8;
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int i = 0; i < MB; ++i) fa[s][i] = frag_a(As, s, i);
#pragma unroll
      for (int j = 0; j < NB; ++j) fb[s][j] = frag_b(Bs, s, j);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };
  // the MFMAs of the fragments in registers
  auto multiply = [&]() {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[s][j], fa[s][i], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  const int n = kt1 - kt0;
  issue(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (wm == 0) {
    for (int t = 0; t < n; ++t) {
      issue(t + 1);
      read_all(t);
      __syncthreads();
      multiply();
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
  } else {
    for (int t = 0; t < n; ++t) {
      issue(t + 1);
      if (t > 0) multiply();
      __syncthreads();
      read_all(t);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
    multiply();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// Workgroup tile BM x BN, WM x WN waves each owning (BM/WM) x (BN/WN).
// How a workgroup's tile reaches C: written (C_STORE), added to C by its one
// writer (C_ADD), or written as a split-K partial (C_SPLIT; split_reduce_kernel
// then sums the partials into C).
enum CMode { C_STORE = 0, C_ADD = 1, C_SPLIT = 2 };

// One workgroup tile: bx, by stand for blockIdx.x, blockIdx.y of a one-product launch.
template <int BM, int BN, int WM, int WN, bool AK, bool BKM, int EPI, typename TC, int CMODE>
__device__ __forceinline__ void gemm_tile(const Params& p, int bx, int by) {
  constexpr int MB = BM / WM / 32, NB = BN / WN / 32;  // 32x32 blocks per wave
  constexpr int kStage = (BM + BN) * 8;                 // uint4 per stage
  // 128 x 128 tiles keep their stages as two distinct objects (the
  // interleaved schedule needs that); 256 x 256 tiles one array of two.
  constexpr bool kW8 = BM == 256 && BN == 256 && WM == 4 && WN == 2;  // mainloop_w8
  constexpr bool kW4M = BM == 256 && BN == 256 && WM == 2 && WN == 2 && EPI != EPI_GELU_GRAD && kUseW4M;
  constexpr bool kSplit = BM != 256 || WM * WN == 4 || kW8;
  __shared__ uint4 smem[kSplit ? kStage : 2 * kStage];
  __shared__ uint4 smem_b[kSplit ? kStage : 1];
  uint4* const stage1 = kSplit ? smem_b : smem + kStage;

  int tm, tn, split;
  if (p.xcd_splits > 0) {
    split_tile_of(bx, p.tiles_m, p.tiles_n, p.xcd_splits, tm, tn, split);
  } else {
    tile_of(bx, p.tiles_m, p.tiles_n, tm, tn);
    split = by;
  }
  const int m0 = tm * BM, n0 = tn * BN;
  const int nkt = total_ktiles(p);
  const int kt0 = split * p.kt_per_split;
  const int kt1 = min(nkt, kt0 + p.kt_per_split);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int L = lane & 31, half = lane >> 5;
  f32x16 acc[kW4M ? 1 : MB][kW4M ? 1 : NB];
  f32x4v acc16[kW4M ? 8 : 1][kW4M ? 8 : 1];
  if constexpr (kW4M)
    mainloop_w4m<AK, BKM>(p, smem, stage1, m0, n0, kt0, kt1, acc16);
  else if constexpr (BM == 256 && BN == 256 && WM == 2 && WN == 4 && AK && !BKM)
    mainloop_pp<AK, BKM>(p, smem, m0, n0, kt0, kt1, acc);  // both stages in smem (kSplit is false)
  else if constexpr (BM == 256 && BN == 256 && WM == 2 && WN == 2)
    mainloop_w4<AK, BKM>(p, smem, stage1, m0, n0, kt0, kt1, acc);
  else if constexpr (kW8)
    mainloop_w8<AK, BKM>(p, smem, stage1, m0, n0, kt0, kt1, acc);
  else
    mainloop<BM, BN, WM, WN, AK, BKM, (BM == 256), kSplit>(p, smem, stage1, m0, n0, kt0, kt1, acc);

  // Epilogue, one 32-row block of the wave's (BM/2) x (BN/2) region at a
  // time: the accumulators go to a wave-private LDS block and come back as
  // whole 16-byte chunks of rows, so each global store instruction writes
  // contiguous row segments; bias and GELU are applied on the way out.
  // Staged as bf16 only for a plain bf16 output, else as fp32 (so the bias
  // is added before the one rounding to the output type).
  using S = typename std::conditional<std::is_same<TC, bf16_t>::value && EPI == EPI_NONE, bf16_t, float>::type;
  constexpr int NW = BN / WN;                // columns per wave
  constexpr int RB = NW * int(sizeof(S));    // staged bytes per row
  constexpr int CQ = RB / 16;                // 16-byte chunks per row
  constexpr int EPC = 16 / int(sizeof(S));   // elements per chunk
  constexpr int RPI = 64 / CQ;               // rows per read instruction
  // (eight-wave 256 x 256 tiles: waves 0-3 stage in the first operand stage, 4-7 in the second)
  constexpr int kStWaves = kW8 ? 4 : WM * WN;
  static_assert(32 * RB * kStWaves <= int(sizeof(smem)), "staging fits in the operand stages");
  unsigned char* stage = reinterpret_cast<unsigned char*>(kW8 && wave >= 4 ? stage1 : smem) + (wave % kStWaves) * 32 * RB;
  const int row0 = m0 + wm * (BM / WM), col0 = n0 + wn * NW;
  // A lane reads back the same columns for every row: col0 + (lane % CQ) * EPC.
  const int qc = lane % CQ;
  const int ncol = col0 + qc * EPC;
  float4 bq = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU) {
    if (ncol < p.N) bq = *reinterpret_cast<const float4*>(p.bias + ncol);
  }
  // The GELU gradient's pre-activations (bf16) of block i+1 stream straight
  // into LDS (unswizzled [32 rows][NW]) while block i is written out.
  constexpr int PB = 32 * NW * 2;  // bytes per pre-activation block and wave
  static_assert(EPI != EPI_GELU_GRAD || (!kW8 && 2 * PB * WM * WN <= kStage * 16), "aux staging");
  unsigned char* pstage = reinterpret_cast<unsigned char*>(stage1) + wave * 2 * PB;
  Operand oaux;
  if constexpr (EPI == EPI_GELU_GRAD) oaux = make_operand(p.aux, p.ldaux, p.aux_span);
  auto fetch_pre = [&](int i) {
    if constexpr (EPI == EPI_GELU_GRAD) {
      constexpr int kChunksRow = NW * 2 / 16;  // 16-byte chunks per row
#pragma unroll
      for (int u = 0; u < PB / 1024; ++u) {
        const int chunk = u * 64 + lane;
        const int r = chunk / kChunksRow, q = chunk % kChunksRow;
        const uint32_t off = static_cast<uint32_t>(row0 + i * 32 + r) * oaux.ld2 + static_cast<uint32_t>(col0 + q * 8) * 2u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            oaux.rsrc, (__attribute__((address_space(3))) void*)(pstage + (i & 1) * PB + u * 1024), 16, off, 0, 0, 0);
      }
    }
  };
  fetch_pre(0);
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    if constexpr (kW4M) {
      // 16 x 16 blocks: lane l holds row 16 a + (l & 15), columns 16 J + 4 (l >> 4) .. + 3
      const int hq = lane >> 4;
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int r = 16 * a + (lane & 15);
#pragma unroll
        for (int J = 0; J < 8; ++J) {
          const int c = 16 * J + 4 * hq;
          f4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x.v[e] = acc16[2 * i + a][J][e];
          if constexpr (sizeof(S) == 4) {
            const int q = c / 4;
            io4<float>::store(reinterpret_cast<float*>(stage + r * RB + ((q ^ (r % CQ)) * 16)), x);
          } else {
            const int q = c / 8;
            io4<bf16_t>::store(reinterpret_cast<bf16_t*>(stage + r * RB + ((q ^ (r % CQ)) * 16) + 8 * (hq & 1)), x);
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c = j * 32 + 8 * g + 4 * half;  // column within the wave's region
          f4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x.v[e] = acc[i][j][4 * g + e];
          if constexpr (sizeof(S) == 4) {
            const int q = c / 4;
            io4<float>::store(reinterpret_cast<float*>(stage + L * RB + ((q ^ (L % CQ)) * 16)), x);
          } else {
            const int q = c / 8;
            io4<bf16_t>::store(reinterpret_cast<bf16_t*>(stage + L * RB + ((q ^ (L % CQ)) * 16) + 8 * half), x);
          }
        }
      }
    }
    if constexpr (EPI == EPI_GELU_GRAD) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (i + 1 < MB) fetch_pre(i + 1);
    {
      // The GELU epilogues stay runtime loops (unrolled they are more code
      // than the instruction cache holds); the others are unrolled.
      constexpr int kStoreUnroll = (EPI == EPI_BIAS_GELU || EPI == EPI_GELU_GRAD) ? 2 : 32;
#pragma unroll kStoreUnroll
      for (int t = 0; t < 32 / RPI; ++t) {
        const int r = t * RPI + lane / CQ;
        const int m = row0 + i * 32 + r, n = ncol;
        const uint4 raw = *reinterpret_cast<const uint4*>(stage + r * RB + ((qc ^ (r % CQ)) * 16));
        if (m >= p.M || n >= p.N) continue;
        TC* cp = CMODE == C_SPLIT
                     ? reinterpret_cast<TC*>(p.part + (static_cast<int64_t>(split) * p.M + m) * p.N + n)
                     : static_cast<TC*>(p.C) + static_cast<int64_t>(m) * p.ldc + n;
        if constexpr (sizeof(S) == 4) {
          f4 x;
          x.v[0] = __uint_as_float(raw.x); x.v[1] = __uint_as_float(raw.y);
          x.v[2] = __uint_as_float(raw.z); x.v[3] = __uint_as_float(raw.w);
          if (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU) {
            x.v[0] += bq.x; x.v[1] += bq.y; x.v[2] += bq.z; x.v[3] += bq.w;
          }
          if (EPI == EPI_BIAS_GELU) {
            // aux = bf16(acc + bias), the pre-activation; C = gelu of it
            io4<bf16_t>::store(p.aux + static_cast<int64_t>(m) * p.ldaux + n, x);
#pragma unroll
            for (int e = 0; e < 4; ++e) x.v[e] = gelu(round_bf16(x.v[e]));
          }
          if constexpr (EPI == EPI_GELU_GRAD) {
            const uint2 w = *reinterpret_cast<const uint2*>(pstage + (i & 1) * PB + r * (NW * 2) + qc * 8);
            x.v[0] *= gelu_grad(__uint_as_float(w.x << 16));
            x.v[1] *= gelu_grad(__uint_as_float(w.x & 0xffff0000u));
            x.v[2] *= gelu_grad(__uint_as_float(w.y << 16));
            x.v[3] *= gelu_grad(__uint_as_float(w.y & 0xffff0000u));
          }
          if constexpr (CMODE == C_ADD) {
            const f4 old = io4<float>::load(reinterpret_cast<const float*>(cp));
#pragma unroll
            for (int e = 0; e < 4; ++e) x.v[e] = old.v[e] + x.v[e];
          }
          if constexpr (EPI == EPI_GELU_GRAD || EPI == EPI_SR)  // gradients: stochastic rounding (mg_common.h)
            io4<TC>::store_grad(cp, x, static_cast<uint32_t>(static_cast<int64_t>(m) * p.N + n), 0x9e5bu);
          else
            io4<TC>::store(cp, x);
        } else {
          *reinterpret_cast<uint4*>(cp) = raw;
        }
      }
    }
    __syncthreads();
  }
}

template <int BM, int BN, int WM, int WN, bool AK, bool BKM, int EPI, typename TC, int CMODE>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(Params p) {
  gemm_tile<BM, BN, WM, WN, AK, BKM, EPI, TC, CMODE>(p, blockIdx.x, blockIdx.y);
}

// Two K-split products in one launch (the FeedForward's two weight
// gradients): workgroups [0, wgs0) run p0's (tile, split) pairs, the rest
// p1's, each laid out by split_tile_of. wgs0 is a multiple of 8, so a
// workgroup's XCD is the same as in a launch of its product alone. One
// launch fills the CUs with half the splits per product, so half the
// partial tiles are written and summed.
template <int BM, int BN, int WM, int WN, bool AK, bool BKM>
__global__ __launch_bounds__(64 * WM * WN) void gemm_pair_kernel(Params p0, Params p1, int wgs0) {
  const int bx = blockIdx.x;
  if (bx < wgs0) gemm_tile<BM, BN, WM, WN, AK, BKM, EPI_NONE, float, C_SPLIT>(p0, bx, 0);
  else gemm_tile<BM, BN, WM, WN, AK, BKM, EPI_NONE, float, C_SPLIT>(p1, bx - wgs0, 0);
}

// ---------------------------------------------------------------- persistent products
//
// Products with more 256 x 256 tiles than CUs and a bf16 output run one
// workgroup per CU that walks its tiles (pid = blockIdx.x, + gridDim.x, ...).
// A workgroup per tile ends each tile exposed: the epilogue, the workgroup's
// exit and the next workgroup's first k-tile load all run with the matrix
// cores idle (measured: the 1024-tile FeedForward product runs its MFMAs 53%
// of the time against 68% for the 256-tile product of equal flops). Here the
// last k-tile of a tile prefetches the next tile's first k-tile into the
// other stage as the k-loop prefetches any k-tile, the epilogue stages its
// bf16 rows in the stage the last k-tile was read from, and its global stores
// drain while the next tile multiplies.
// The main loop is mainloop_w8's (eight waves, 64 x 128 each, waves 0-3 load),
// with the operand offsets taken relative to the tile origin (a scalar per
// tile). It needs an even k-tile count, so that every tile starts from stage
// `sa` and ends in `sb`.
// Epilogue math (bias, GELU, stochastic rounding) is done in registers on the
// lane's own 4 consecutive columns of a row, so the staging is bf16: 8 KB per
// wave, one stage for all eight waves.
template <bool AK, bool BKM, int EPI>
__global__ __launch_bounds__(512) void gemm_persist_kernel(Params p) {
  constexpr int S = BK / 16;
  constexpr int kLoaders = 4;
  constexpr int NL = kW4Loads * 4 / kLoaders;
  constexpr int kStageA = kW4Rows * 8;  // uint4 of the A tile (B follows)
  constexpr int kStage = 2 * kStageA;
  __shared__ uint4 sa[kStage];
  __shared__ uint4 sb[kStage];
  // the bias of a tile's 256 columns, double-buffered by tile parity: wave 0
  // loads the next tile's into LDS during the current epilogue, and its wait
  // for the next k-tile's loads covers that load too
  constexpr bool kBias = EPI == EPI_BIAS || EPI == EPI_BIAS_GELU;
  __shared__ float4 s_bias[kBias ? 2 : 1][64];
  const int ntiles = p.tiles_m * p.tiles_n;
  const int n = total_ktiles(p);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const Operand oa = make_operand(p.A, p.lda, p.a_span);
  const Operand ob = make_operand(p.B, p.ldb, p.b_span);
  W4Operand<AK> A;
  W4Operand<BKM> B;
  A.template init<NL>(oa, 0, wm * 64, wave % kLoaders, lane);
  B.template init<NL>(ob, 0, wn * 128, wave % kLoaders, lane);
  // byte shift of tile pid's operand blocks against the tile at the origin
  auto origin = [&](int pid, int& m0, int& n0, uint32_t& ash, uint32_t& bsh) {
    int tm, tn;
    tile_of(pid, p.tiles_m, p.tiles_n, tm, tn);
    m0 = tm * 256;
    n0 = tn * 256;
    ash = AK ? static_cast<uint32_t>(m0) * oa.ld2 : static_cast<uint32_t>(m0) * 2u;
    bsh = BKM ? static_cast<uint32_t>(n0) * ob.ld2 : static_cast<uint32_t>(n0) * 2u;
  };
  // offsets of k-tile t of a tile with shifts (ash, bsh)
  auto koffs = [&](int t, uint32_t ash, uint32_t bsh, uint32_t& ao, uint32_t& bo) {
    int seg = 0, k0 = t * BK;
    if (p.hilo) {
      seg = t / p.nkt_seg;
      k0 = (t - seg * p.nkt_seg) * BK;
    }
    ao = A.koff(k0, seg == 1 ? p.K : 0, oa.ld2) + ash;
    bo = B.koff(k0, seg == 2 ? p.K : 0, ob.ld2) + bsh;
  };
  bf16x8 af[2][2], bfr[2][4];
  auto read_step = [&](const uint4* st, int s, int buf) {
    af[buf][0] = A.frag(st, s, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[buf][j] = B.frag(st + kStageA, s, j);
    af[buf][1] = A.frag(st, s, 1);
  };
  f32x16 acc[2][4];
  auto mfma_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[buf][j], af[buf][i], acc[i][j], 0, 0, 0);
  };
  constexpr int NR = 2 * W4Operand<AK>::kReadsPerBlock + 4 * W4Operand<BKM>::kReadsPerBlock;

  int pid = blockIdx.x;
  int m0, n0;
  uint32_t ash, bsh;
  origin(pid, m0, n0, ash, bsh);
  __amdgpu_buffer_rsrc_t bias_rsrc;
  if constexpr (kBias)
    bias_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.bias), static_cast<short>(0), p.N * 4, 0x00020000);
  auto load_bias = [&](int par, int col0) {  // wave 0; columns past N read as zero
    if constexpr (kBias)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(bias_rsrc, (__attribute__((address_space(3))) void*)(&s_bias[par][0]), 16,
                                               static_cast<uint32_t>(col0 + 4 * lane) * 4u, 0, 0, 0);
  };
  if (wave == 0) load_bias(0, n0);
  if (wave < kLoaders) {  // the first tile's first k-tile
    uint32_t ao, bo;
    koffs(0, ash, bsh, ao, bo);
#pragma unroll
    for (int i = 0; i < NL; ++i) A.template load<NL>(sa, wave, i, ao);
#pragma unroll
    for (int i = 0; i < NL; ++i) B.template load<NL>(sa + kStageA, wave, i, bo);
  }
  for (int it = 0;; ++it) {
    const bool first = it == 0;
    const int next = pid + static_cast<int>(gridDim.x);
    const bool has_next = next < ntiles;
    int m1 = 0, n1 = 0;
    uint32_t ash1 = 0, bsh1 = 0;
    if (has_next) origin(next, m1, n1, ash1, bsh1);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    // The loop once per role (loading waves 0-3, the others), as in mainloop_w8.
    auto run = [&](auto role) __attribute__((always_inline)) {
      constexpr bool kLoad = decltype(role)::value;
      // The first tile waits for its first k-tile here; a later tile's first
      // k-tile was waited for at the previous tile's last k-step (waiting
      // again would also wait for the epilogue's stores).
      if (kLoad && first) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // this tile's first k-tile is in sa; the previous epilogue is done with sb
      read_step(sa, 0, 0);
      auto tile = [&](int t, const uint4* cur, uint4* nxt) __attribute__((always_inline)) {
        // prefetch k-tile t + 1 of this tile, else the next tile's first
        // k-tile, else (the last tile) a reload of this k-tile; the loads stay
        // unconditional so that they share one scheduled block with the MFMAs
        uint32_t ao = 0, bo = 0;
        if constexpr (kLoad) {
          if (t + 1 < n) koffs(t + 1, ash, bsh, ao, bo);
          else if (has_next) koffs(0, ash1, bsh1, ao, bo);
          else koffs(t, ash, bsh, ao, bo);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int c = s & 1;
          if constexpr (kLoad) {
            if (s == 0) {
#pragma unroll
              for (int i = 0; i < NL; ++i) A.template load<NL>(nxt, wave, i, ao);
            } else if (s == 1) {
#pragma unroll
              for (int i = 0; i < NL; ++i) B.template load<NL>(nxt + kStageA, wave, i, bo);
            }
          }
          if (s + 1 < S) {
            read_step(cur, s + 1, c ^ 1);
          } else {
            // only the loading waves have loads to wait for (the others' epilogue
            // stores of the previous tile are left to drain)
            if constexpr (kLoad) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();  // k-tile t + 1 is in `nxt` for every wave; every wave is done with `cur`
            read_step(nxt, 0, c ^ 1);
          }
          mfma_step(c);
          if (kLoad && s < 2) interleave<8, NR, NL>();
          else interleave<8, NR, 0>();
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      for (int t = 0; t < n; t += 2) {
        tile(t, sa, sb);
        tile(t + 1, sb, sa);
      }
    };
    if (wave < kLoaders) run(std::true_type{});
    else run(std::false_type{});

    // Epilogue: every wave has passed the last k-tile's barrier, so sb (the
    // last k-tile's stage) is free; sa holds the next tile's first k-tile.
    // Rows row0 + 32 i + L, columns col0 + 32 j + 8 g + 4 half + e of the
    // lane's accumulators go as bf16 into a per-wave 32 x 128 staging block;
    // the non-loading waves 4-7 read back the blocks of waves w and w + 4 as
    // 16-byte row chunks and store them. The loading waves issue no stores,
    // so their wait for the next k-tile's loads does not wait for the stores
    // (one vector-memory counter per wave counts both, in issue order): the
    // output of all CUs, written at the same moment, drains while the next
    // tile multiplies.
    if (wave == 0 && has_next) load_bias((it + 1) & 1, n1);
    {
      constexpr int RB = 256, CQ = RB / 16, RPI = 64 / CQ;
      unsigned char* stg = reinterpret_cast<unsigned char*>(sb) + wave * (32 * RB);
      const int L = lane & 31, half = lane >> 5;
      const int row0 = m0 + wm * 64, col0 = n0 + wn * 128;
      const int qc = lane % CQ;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int c = j * 32 + 8 * g + 4 * half;
            const int col = col0 + c;
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = acc[i][j][4 * g + e];
            if constexpr (kBias) {
              const float4 bq = s_bias[it & 1][(col - n0) / 4];
              x[0] += bq.x; x[1] += bq.y; x[2] += bq.z; x[3] += bq.w;
            }
            uint2 w;
            if constexpr (EPI == EPI_SR) {
              const uint32_t idx = static_cast<uint32_t>(static_cast<int64_t>(row0 + i * 32 + L) * p.N + col);
              w.x = pack_bf16x2_sr(x[0], x[1], idx, 0x9e5bu);
              w.y = pack_bf16x2_sr(x[2], x[3], idx + 2, 0x9e5bu);
            } else {
              w.x = pack_bf16x2(x[0], x[1]);
              w.y = pack_bf16x2(x[2], x[3]);
            }
            const int q = c / 8;
            *reinterpret_cast<uint2*>(stg + L * RB + ((q ^ (L % CQ)) * 16) + 8 * half) = w;
          }
        }
        __syncthreads();
        if (wave >= kLoaders) {
          // BIAS_GELU: the staged values are the pre-activation (aux); C =
          // gelu of them, computed here (a runtime loop: unrolled, the GELU
          // is more code than the instruction cache holds)
#pragma unroll 1
          for (int h = 0; h < 2; ++h) {
            const int src = wave - kLoaders + kLoaders * h;  // waves w, w + 4
            const unsigned char* sst = reinterpret_cast<const unsigned char*>(sb) + src * (32 * RB);
            const int srow = m0 + (src >> 1) * 64 + i * 32, scol = n0 + (src & 1) * 128 + qc * 8;
            constexpr int kUnroll = EPI == EPI_BIAS_GELU ? 1 : 32 / RPI;
#pragma unroll kUnroll
            for (int t = 0; t < 32 / RPI; ++t) {
              const int r = t * RPI + lane / CQ;
              const int m = srow + r;
              const uint4 raw = *reinterpret_cast<const uint4*>(sst + r * RB + ((qc ^ (r % CQ)) * 16));
              if (m < p.M && scol < p.N) {
                if constexpr (EPI == EPI_BIAS_GELU) {
                  *reinterpret_cast<uint4*>(p.aux + static_cast<int64_t>(m) * p.ldaux + scol) = raw;
                  const uint32_t wi[4] = {raw.x, raw.y, raw.z, raw.w};
                  uint32_t wo[4];
#pragma unroll
                  for (int e = 0; e < 4; ++e)
                    wo[e] = pack_bf16x2(gelu(__uint_as_float(wi[e] << 16)), gelu(__uint_as_float(wi[e] & 0xffff0000u)));
                  *reinterpret_cast<uint4*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(m) * p.ldc + scol) =
                      make_uint4(wo[0], wo[1], wo[2], wo[3]);
                } else {
                  *reinterpret_cast<uint4*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(m) * p.ldc + scol) = raw;
                }
              }
            }
          }
        }
        __syncthreads();
      }
    }
    if (!has_next) break;
    pid = next;
    m0 = m1;
    n0 = n1;
    ash = ash1;
    bsh = bsh1;
  }
}

// Persistent products on the four-wave 16x16x32 pipeline (W4MPipe): one
// workgroup per CU walks tiles pid, pid + gridDim.x, ... as one continuous
// k-tile pipeline: the last k-steps of a tile load the next tile's first two
// k-tiles and read its first fragments, so a tile's epilogue runs with the
// next tile's operands already in LDS. Needs an even k-tile count (every tile
// then starts in stage sa).
// Epilogue, per wave and in registers: bias, then bf16 rounding (round to
// nearest, or stochastic for a gradient), 16 rows at a time into a
// wave-private staging block, read back as 16-byte row chunks and stored (for
// BIAS_GELU the staged values are the pre-activation: it is stored to aux and
// C = gelu of it). The staging is the wave's own, so the epilogue needs no
// workgroup barrier, and it is beside the operand stages, which hold the next
// tile's k-tiles.
// kPrefix: only the tiles of output columns below p.hilo_cols are hi/lo
// products (three K segments), the others take the first segment alone
// (mg_gemm_hilo_prefix); the tile ids [0, T1) walk the first kind, then the
// others, each laid out as tile_of lays out a product of its own.
template <bool AK, bool BKM, int EPI, bool kPrefix = false>
__global__ __launch_bounds__(256) void gemm_persist_w4m_kernel(Params p) {
  using Pipe = W4MPipe<AK, BKM>;
  constexpr int kStage = 2 * Pipe::kStageA;
  constexpr bool kBias = EPI == EPI_BIAS || EPI == EPI_BIAS_GELU;
  __shared__ uint4 sa[kStage];
  __shared__ uint4 sb[kStage];
  // per wave: 16 rows x 128 bf16 (16 chunks of 16 bytes a row). Indexed
  // through this array itself (not a byte pointer into it): the compiler then
  // tells it apart from the operand stages and does not wait for the next
  // tile's direct-to-LDS loads before the epilogue's LDS writes.
  __shared__ uint2 stg2[4 * 512];
  __shared__ float4 s_bias[kBias ? 2 : 1][64];
  // BIAS_GELU: C = gelu(aux) by table lookup in the epilogue
  constexpr bool kGelu = EPI == EPI_BIAS_GELU;
  __shared__ uint16_t s_gelu[kGelu ? kGeluLutN : 1];
  const int ntiles = p.tiles_m * p.tiles_n;
  const int tn1 = kPrefix ? p.hilo_cols / 256 : p.tiles_n;
  const int T1 = p.tiles_m * tn1;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  Pipe P;
  P.init(p, wave, lane);
  f32x4v acc[8][8];
  int pid = blockIdx.x;
  auto origin = [&](int id, int& m0, int& n0) {
    int tm, tn;
    if (!kPrefix || id < T1) {
      tile_of(id, p.tiles_m, tn1, tm, tn);
    } else {
      tile_of(id - T1, p.tiles_m, p.tiles_n - tn1, tm, tn);
      tn += tn1;
    }
    m0 = tm * 256;
    n0 = tn * 256;
  };
  int m0, n0;
  origin(pid, m0, n0);
  int n = total_ktiles(p);
  if constexpr (kPrefix) {
    n = __builtin_amdgcn_readfirstlane(n0 < p.hilo_cols ? 3 * p.nkt_seg : p.nkt_seg);
    P.set_hilo(p, n0 < p.hilo_cols);
  }
  uint32_t ar = P.aorg(m0), br = P.borg(n0);
  __amdgpu_buffer_rsrc_t bias_rsrc;
  if constexpr (kBias)
    bias_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.bias), static_cast<short>(0), p.N * 4, 0x00020000);
  auto load_bias = [&](int par, int col0) {  // wave 0; columns past N read as zero
    if constexpr (kBias)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(bias_rsrc, (__attribute__((address_space(3))) void*)(&s_bias[par][0]), 16,
                                               static_cast<uint32_t>(col0 + 4 * lane) * 4u, 0, 0, 0);
  };
  if (wave == 0) load_bias(0, n0);
  {  // the first tile: k-tiles 0 and 1 in flight, k-tile 0 waited for, its first fragments read
    uint32_t ao, bo;
    P.koffs(0, ao, bo);
    P.load_tile(sa, ao, bo, ar, br);
    P.koffs(1 % n, ao, bo);
    P.load_tile(sb, ao, bo, ar, br);
  }
  if constexpr (kGelu) gelu_lut_fill(s_gelu);  // under the first loads; the barrier below publishes it
  asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  __syncthreads();
  P.read_all(sa, 0, 0);
  for (int it = 0;; ++it) {
    const int next = pid + static_cast<int>(gridDim.x);
    const bool has_next = next < ntiles;
    int m1 = m0, n1 = n0;
    if (has_next) origin(next, m1, n1);
    const uint32_t ar1 = P.aorg(m1), br1 = P.borg(n1);
    // k-step 0 of k-tile 0 (acc = product), reading its k-step 1 fragments;
    // then k-tile 1 is waited for (with the previous tile's epilogue stores)
    P.template kstep<0, true, false, true>(acc, sa, 1, sa, 0, 0, ar, br);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // units t = 0 .. n - 2 (as in mainloop_w4m): k-step 1 of k-tile t loading
    // k-tile t + 2 (the next tile's k-tile 0 for t = n - 2), k-step 0 of
    // k-tile t + 1
    auto unit = [&](int t, uint4* cur, const uint4* nxt) __attribute__((always_inline)) {
      P.opaque();
      uint32_t lo, lb, la = ar, lbr = br;
      if (t + 2 < n) {
        P.koffs(t + 2, lo, lb);
      } else {
        P.koffs(0, lo, lb);
        la = ar1;
        lbr = br1;
      }
      P.template kstep<1, true, true, false>(acc, nxt, 0, cur, lo, lb, la, lbr);
      P.template kstep<0, true, false, false>(acc, nxt, 1, cur, 0, 0, ar, br);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    };
    int t = 0;
    for (; t + 3 < n; t += 2) {
      unit(t, sa, sb);
      unit(t + 1, sb, sa);
    }
    unit(t, sa, sb);  // t = n - 2
    // k-step 1 of the last k-tile (stage sb): loads the next tile's k-tile 1
    // into sb and reads its k-tile 0's first fragments from sa (the last
    // tile reloads its own k-tile 1, harmlessly)
    {
      P.opaque();
      uint32_t lo, lb;
      P.koffs(1 % n, lo, lb);
      P.template kstep<1, true, true, false>(acc, sa, 0, sb, lo, lb, ar1, br1);
    }
    mfma16_agpr_drain(acc);

    // epilogue (this wave's 128 x 128 block of the tile). The lane index is
    // made opaque here, so that the lane-dependent addresses below are
    // computed per tile, not hoisted out of the tile loop and held in
    // registers through the k-loop.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int rl = ln & 15, hq = ln >> 4;
    const int row0 = m0 + wm * 128, col0 = wn * 128;  // col0 within the tile
    uint32_t excmask = 0;  // GELU: bit 4 I + u, chunk (I, u) has a value outside the table
    float4 bq[8];  // the bias of the lane's 4 columns of each 16-column block
    if constexpr (kBias) {
#pragma unroll
      for (int J = 0; J < 8; ++J) bq[J] = s_bias[it & 1][(col0 + 16 * J + 4 * hq) / 4];
    }

#pragma unroll
    for (int I = 0; I < 8; ++I) {
      __builtin_amdgcn_sched_barrier(0);  // block I's accumulator reads stay here (hoisted, they spill)
#pragma unroll
      for (int J = 0; J < 8; ++J) {
        const int c = col0 + 16 * J + 4 * hq;  // tile column of the lane's first value
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = acc[I][J][e];
        if constexpr (kBias) {
          x[0] += bq[J].x; x[1] += bq[J].y; x[2] += bq[J].z; x[3] += bq[J].w;
        }
        uint2 w;
        if constexpr (EPI == EPI_SR) {
          const uint32_t idx = static_cast<uint32_t>(static_cast<int64_t>(row0 + 16 * I + rl) * p.N + n0 + c);
          w.x = pack_bf16x2_sr(x[0], x[1], idx, 0x9e5bu);
          w.y = pack_bf16x2_sr(x[2], x[3], idx + 2, 0x9e5bu);
        } else {
          w.x = pack_bf16x2(x[0], x[1]);
          w.y = pack_bf16x2(x[2], x[3]);
        }
        // row rl, 16-byte chunk (2 J + (hq >> 1)) ^ rl, half hq & 1
        stg2[wave * 512 + rl * 32 + ((((2 * J) | (hq >> 1)) ^ rl) << 1) + (hq & 1)] = w;
      }
      // read back 4 rows x 256 bytes per instruction and store
      const int cq = ln & 15;
      const int ncol = n0 + col0 + 8 * cq;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int rr = 4 * u + hq;
        const uint4 raw = reinterpret_cast<const uint4*>(stg2)[wave * 256 + rr * 16 + (cq ^ rr)];
        const int m = row0 + 16 * I + rr;
        if (m < p.M && ncol < p.N) {
          if constexpr (kGelu) {
            store_aux(p.aux + static_cast<int64_t>(m) * p.ldaux + ncol, raw);
            bool exc = false;
            const uint4 y = gelu_lut_chunk(raw, s_gelu, exc);
            *reinterpret_cast<uint4*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(m) * p.ldc + ncol) = y;
            excmask |= exc ? 1u << (4 * I + u) : 0u;
          } else {
            *reinterpret_cast<uint4*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(m) * p.ldc + ncol) = raw;
          }
        }
      }
    }
    if constexpr (kGelu) {
      // the chunks with a value outside the table (rare), by gelu() itself,
      // from the aux chunks the lane stored above (the same thread's store,
      // waited for). Out of the unrolled block loop: inline there, the exact
      // path's code made the compiler spill.
      if (__builtin_amdgcn_ballot_w64(excmask != 0) != 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const int ncol = n0 + col0 + 8 * (ln & 15);
#pragma unroll 1
        for (int q = 0; q < 32; ++q) {
          if ((excmask >> q) & 1u) {
            const int m = row0 + 4 * q + hq;  // block I = q / 4, rows 4 u + hq of it
            const uint4 raw = *reinterpret_cast<const uint4*>(p.aux + static_cast<int64_t>(m) * p.ldaux + ncol);
            *reinterpret_cast<uint4*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(m) * p.ldc + ncol) =
                gelu_exact_chunk(raw);
          }
        }
      }
    }
    // the next tile's bias, once this epilogue's LDS accesses are issued (an LDS
    // access after a direct-to-LDS load the compiler cannot tell apart from it
    // waits for every load in flight)
    if (wave == 0 && has_next) load_bias((it + 1) & 1, n1);
    if (!has_next) break;
    pid = next;
    m0 = m1;
    n0 = n1;
    ar = ar1;
    br = br1;
    if constexpr (kPrefix) {
      // the next tile's k-tiles 0 and 1 (loaded above) lie in the first K segment
      // whatever its mode; its mode sets where its later k-tiles come from
      n = __builtin_amdgcn_readfirstlane(n0 < p.hilo_cols ? 3 * p.nkt_seg : p.nkt_seg);
      P.set_hilo(p, n0 < p.hilo_cols);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last tile's spare loads land before the LDS is released
}

// ---------------------------------------------------------------- loss head
//
// Streaming cross-entropy head: logits = E W^T for 64 rows at a time with
// all V (<= 256) classes in one workgroup tile, then, from LDS, per row
//   lse = max + log(sum exp(l - max)),  loss = lse - l[label],
//   dlogits = (softmax - onehot(label)) * scale   (bf16),
// so the fp32 logits never reach HBM. Reference mingru/minLM.py:138,146-149
// (to_logits, F.cross_entropy with mean reduction); loss_part[b] = sum of
// the row losses of workgroup b.
constexpr int kCeRows = 64;

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

// Four-stage k-loop of the loss head's product (64 x 256 tile, four waves of
// 64 x 64): the loads of k-tile t + 3 go out while tile t is multiplied, so
// three tiles' loads (120 KB) are in flight. With K = 1024 the product has
// only 16 short k-tiles (16 MFMAs per wave each), and every workgroup reads
// all of W from L2 (512 KB per 64 rows): the product is bound by how many
// bytes each CU keeps in flight against the L2 latency, so the four stages
// fill the whole 160 KB of LDS. The stages are four distinct __shared__
// arrays, run in turns of four so each is static (an LDS read then waits only
// for the loads into its own stage).
__device__ __forceinline__ void ce_mainloop4(const Params& p, uint4* s0, uint4* s1, uint4* s2, uint4* s3, int m0,
                                             int n, f32x16 (&acc)[2][2]) {
  constexpr int BM = kCeRows, BN = 256, MB = 2, NB = 2, T = 256, S = BK / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  const Operand oa = make_operand(p.A, p.lda, p.a_span);
  const Operand ob = make_operand(p.B, p.ldb, p.b_span);
  Loader<BM, true, T> la;
  Loader<BN, true, T> lb;
  constexpr int kLoads = decltype(la)::kPerWave + decltype(lb)::kPerWave;  // load instructions per tile and wave
  auto issue_to = [&](int t, uint4* st) {  // tiles past n read as zero
    const KTile kt = ktile(p, t, n);
    la.load(oa, st, m0, p.M, kt.k0, kt.kmax, kt.aofs);
    lb.load(ob, st + BM * 8, 0, p.N, kt.k0, kt.kmax, kt.bofs);
  };
  int arow[MB], brow[NB];
#pragma unroll
  for (int i = 0; i < MB; ++i) arow[i] = i * 32;
#pragma unroll
  for (int j = 0; j < NB; ++j) brow[j] = wave * 64 + j * 32;
  issue_to(0, s0);
  issue_to(1, s1);
  issue_to(2, s2);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kLoads) : "memory");  // tile 0 has landed
  __builtin_amdgcn_s_barrier();
  bf16x8 af[2][MB], bfr[2][NB];
  auto tile = [&](int t, const uint4* cur, uint4* fill) __attribute__((always_inline)) {
    issue_to(t + 3, fill);  // fill held tile t - 1, which every wave finished before the last barrier
    const uint4* Bs = cur + BM * 8;
#pragma unroll
    for (int i = 0; i < MB; ++i) af[0][i] = read_frag<BM, true>(cur, arow[i], 0, lane);
#pragma unroll
    for (int j = 0; j < NB; ++j) bfr[0][j] = read_frag<BN, true>(Bs, brow[j], 0, lane);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int c = s & 1;
      if (s + 1 < S) {
#pragma unroll
        for (int i = 0; i < MB; ++i) af[c ^ 1][i] = read_frag<BM, true>(cur, arow[i], s + 1, lane);
#pragma unroll
        for (int j = 0; j < NB; ++j) bfr[c ^ 1][j] = read_frag<BN, true>(Bs, brow[j], s + 1, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[c][j], af[c][i], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Tile t + 1 has landed (t + 2 and t + 3 may still fly). A bare
    // s_barrier, not __syncthreads(), whose fence would wait for every load
    // in flight: this wave's loads into t + 1's stage are complete by the
    // vmcnt wait, every wave's reads of tile t were consumed by its MFMAs,
    // and the barrier makes both hold for the whole workgroup.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kLoads) : "memory");
    __builtin_amdgcn_s_barrier();
  };
  int t = 0;
  for (; t + 3 < n; t += 4) {
    tile(t, s0, s3);
    tile(t + 1, s1, s0);
    tile(t + 2, s2, s1);
    tile(t + 3, s3, s2);
  }
  if (t < n) tile(t, s0, s3);
  if (t + 1 < n) tile(t + 1, s1, s0);
  if (t + 2 < n) tile(t + 2, s2, s1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the zero-reading loads past n
  __syncthreads();
}

__global__ __launch_bounds__(256) void logits_ce_kernel(Params p, const int64_t* __restrict__ labels,
                                                        bf16_t* __restrict__ dlogits, int64_t ldd,
                                                        float* __restrict__ loss_part, int* __restrict__ bad_label,
                                                        float scale) {
  constexpr int BM = kCeRows, BN = 256, WM = 1, WN = 4;
  constexpr int MB = BM / WM / 32, NB = BN / WN / 32;
  constexpr int kStage = (BM + BN) * 8;
  __shared__ uint4 st0[kStage], st1[kStage], st2[kStage], st3[kStage];
  float* const s_loss = reinterpret_cast<float*>(st2);  // after the product (st2 is not part of the logits tile)
  // the fp32 logits tile after the product: rows [0, kRows0) in st0, the rest in st1
  constexpr int kRows0 = kStage * 16 / (BN * 4);
  static_assert(BM - kRows0 <= kRows0, "logits tile fits in two stages");
  auto tile_row = [&](int r) -> float* {
    return r < kRows0 ? reinterpret_cast<float*>(st0) + r * BN : reinterpret_cast<float*>(st1) + (r - kRows0) * BN;
  };

  const int m0 = blockIdx.x * BM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int L = lane & 31, half = lane >> 5;
  // this wave's 16 labels, one per lane, loaded before the product so their
  // latency hides under it (read per row, each would be a dependent load)
  int64_t my_lab = 0;
  {
    const int64_t row = static_cast<int64_t>(m0) + wave * (BM / 4) + lane;
    if (lane < BM / 4 && row < p.M) my_lab = labels[row];
  }
  f32x16 acc[MB][NB];
  static_assert(MB == 2 && NB == 2 && WM == 1 && WN == 4, "ce_mainloop4's tile");
  ce_mainloop4(p, st0, st1, st2, st3, m0, (p.K + BK - 1) / BK, acc);

  // logits tile [64][256] fp32 in LDS, 16-byte chunk c of row r at c ^ (r & 63)
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = i * 32 + L;
        const int c = wave * (BN / WN / 4) + j * 8 + 2 * g + half;
        f4 x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x.v[e] = acc[i][j][4 * g + e];
        io4<float>::store(tile_row(r) + ((c ^ (r & 63)) * 4), x);
      }
  __syncthreads();

  // Softmax tail, all 16 rows of the wave at once: lane 4 rl + q holds classes
  // 64 q .. 64 q + 63 of the wave's row rl (register x[4 k + e] is class
  // 64 q + 4 kk(k) + e, kk(k) = (k + 2 q + 4 (r & 1)) & 15: staggered so the 8
  // lanes of each LDS read phase, two rows by four quarters, hit distinct banks);
  // the row's max and sum combine over its four lanes.
  const int V = p.N;
  const int rl = lane >> 2, q = lane & 3;
  const int r = wave * (BM / 4) + rl;
  const int64_t row = static_cast<int64_t>(m0) + r;
  const int64_t lab = __shfl(my_lab, rl, 64);
  const int stag = 2 * q + 4 * (r & 1);
  const bool lab_ok = lab >= 0 && lab < V;
  float x[64];
  float m = -INFINITY;
  // kFull: V == 256, no class past V to mask
  auto load_row = [&](auto full_tag) {
    constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int c = q * 16 + ((k + stag) & 15);  // this lane's chunk k: classes 4c .. 4c + 3
      const f4 v = io4<float>::load(tile_row(r) + ((c ^ (r & 63)) * 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float l = (kFull || 4 * c + e < V) ? v.v[e] : -INFINITY;
        x[4 * k + e] = l;
        m = fmaxf(m, l);
      }
    }
  };
  if (V == 256)
    load_row(std::true_type{});
  else
    load_row(std::false_type{});
  // the label's logit, read once by each of the row's four lanes
  const int labi = lab_ok ? static_cast<int>(lab) : 0;
  const float picked = lab_ok ? tile_row(r)[((labi >> 2) ^ (r & 63)) * 4 + (labi & 3)] : 0.0f;
  m = fmaxf(m, __shfl_xor(m, 1, 64));
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  // e^(l - m) as 2^(l log2(e) - mc) with mc = m log2(e) rounded once: the
  // rounding of mc scales every term of the row alike, and the log-sum-exp
  // below adds back the same mc (classes past V: 2^-inf = 0)
  const float mc = m * kLog2e;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    x[i] = exp2_raw(__builtin_fmaf(x[i], kLog2e, -mc));
    sum += x[i];
  }
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  const bool live = row < p.M;
  float lsum = 0.0f;
  if (live && q == 0) {
    lsum = logf(sum) + mc * 0.69314718055994531f - picked;
    if (!lab_ok && bad_label) atomicOr(bad_label, 1);
  }
  if (live) {
    const float s = scale / sum;  // dlogits = softmax * scale - onehot * scale
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // chunks 2u, 2u + 1 are classes 8 consecutive from 4 c0 (stag is even)
      const int c0 = q * 16 + ((2 * u + stag) & 15);
      if (4 * c0 >= V) continue;
      fv<8> d;
#pragma unroll
      for (int e = 0; e < 8; ++e) d.v[e] = __builtin_fmaf(x[8 * u + e], s, 4 * c0 + e == lab ? -scale : 0.0f);
      // stochastic rounding of the bf16 gradient (mg_common.h): round-to-nearest errors of
      // this near-uniform softmax repeat across the rows of a label
      iov<bf16_t, 8>::store_grad(dlogits + row * ldd + 4 * c0, d, static_cast<uint32_t>(row * V + 4 * c0), 0x8d4au);
    }
  }
  lsum = wave_sum(lsum);
  if (lane == 0) s_loss[wave] = lsum;
  __syncthreads();
  if (threadIdx.x == 0) loss_part[blockIdx.x] = s_loss[0] + s_loss[1] + s_loss[2] + s_loss[3];
}

// The split-K reduction reads each partial once and writes a weight gradient
// the optimizer reads at the end of the step: both carry the non-temporal hint
// (cfg3 step 11.19 -> 11.14 ms).
typedef float f32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4 load4_stream(const float* q) {
  const f32x4_nt x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(q));
  f4 r; r.v[0] = x[0]; r.v[1] = x[1]; r.v[2] = x[2]; r.v[3] = x[3];
  return r;
}
__device__ __forceinline__ void store4_stream(float* q, const f4& r) {
  const f32x4_nt x = {r.v[0], r.v[1], r.v[2], r.v[3]};
  __builtin_nontemporal_store(x, reinterpret_cast<f32x4_nt*>(q));
}

// C[m, n] (+)= sum over the S split partials, added in split order.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part, int S, int M, int N,
                                                           float* __restrict__ C, int64_t ldc, int accumulate) {
  const int64_t n4 = static_cast<int64_t>(M) * (N / 4);
  const int64_t slice = static_cast<int64_t>(M) * N;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n4;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = i / (N / 4), n = (i % (N / 4)) * 4;
    float* cp = C + m * ldc + n;
    f4 sum = accumulate ? io4<float>::load(cp) : io4<float>::fill(0.0f);
    const float* pp = part + m * N + n;
    int s = 0;
    for (; s + 8 <= S; s += 8) {  // eight partials in flight
      f4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = load4_stream(pp + (s + u) * slice);
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum.v[e] += v[u].v[e];
    }
    for (; s + 2 <= S; s += 2) {
      const f4 v0 = load4_stream(pp + s * slice), v1 = load4_stream(pp + (s + 1) * slice);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum.v[e] += v0.v[e];
#pragma unroll
      for (int e = 0; e < 4; ++e) sum.v[e] += v1.v[e];
    }
    for (; s < S; ++s) {
      const f4 v0 = load4_stream(pp + s * slice);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum.v[e] += v0.v[e];
    }
    store4_stream(cp, sum);
  }
}

// C[m, n] = bf16 of the sum over the S split partials (in split order), plus bias[n] when
// given (EPI_BIAS): rounded to nearest, or stochastically with the unsplit epilogue's hash of
// the element index (EPI_SR), so only the fp32 sum's order differs from the unsplit product.
__global__ __launch_bounds__(256) void split_reduce_bf16_kernel(const float* __restrict__ part, int S, int M, int N,
                                                               bf16_t* __restrict__ C, int64_t ldc, int stochastic,
                                                               const float* __restrict__ bias) {
  const int64_t n4 = static_cast<int64_t>(M) * (N / 4);
  const int64_t slice = static_cast<int64_t>(M) * N;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n4;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = i / (N / 4), n = (i % (N / 4)) * 4;
    const float* pp = part + m * N + n;
    f4 sum = io4<float>::fill(0.0f);
    for (int s = 0; s < S; ++s) {
      const f4 v = load4_stream(pp + s * slice);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum.v[e] += v.v[e];
    }
    if (bias) {
      const f4 bv = io4<float>::load(bias + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum.v[e] += bv.v[e];
    }
    bf16_t* cp = C + m * ldc + n;
    if (stochastic)
      io4<bf16_t>::store_grad(cp, sum, static_cast<uint32_t>(m * N + n), 0x9e5bu);
    else
      io4<bf16_t>::store(cp, sum);
  }
}

constexpr int kCUs = 256;

// Tile size and K split of a product (measured on MI355X): 256 x 256 tiles for
// weight gradients (both operands MN-contiguous) of whole 256 x 256 tiles, at
// least 16 of them, K >= 4096, split along K to about one workgroup per CU, and
// for the other layouts when that still gives every CU a tile; everything else
// 128 x 128, split along K (outputs and epilogues that allow it) to about two
// workgroups per CU. `ysplits` is the split count the launch uses (gridDim.y).
struct Plan {
  bool big;
  int tiles, kt_per_split, ysplits;
};

inline Plan plan(int M, int N, int K, bool ak, bool bk, int c_dtype, int epilogue, bool deterministic, bool hilo) {
  Plan pl;
  const int64_t t256 = int64_t((M + 255) / 256) * ((N + 255) / 256);
  const int64_t t128 = int64_t((M + 127) / 128) * ((N + 127) / 128);
  const bool wgrad = !ak && !bk;
  // weight gradients whose output dimensions are multiples of 256 run 256 x 256
  // tiles (half the L2 traffic per flop of 128 x 128), split along K to about
  // one workgroup per CU; with fewer than 16 such tiles (the logits' 256 x 1024:
  // 4 tiles, 64 splits of 4 k-tiles) the splits get too short and their
  // partials too many, and 128 x 128 tiles are faster (measured 27 against 40 us).
  // Below K 4096 (a [1, 2048] chunk's weight gradients, added into .grad) the
  // 128 x 128 tiles need fewer splits or none, so fewer partials to write and add
  // (d1024 expansion-3 optimizer step 348.4 -> 343.7 ms)
#ifndef MG_GEMM_WGRAD128
  const bool wgrad_big = wgrad && M % 256 == 0 && N % 256 == 0 && t256 >= 16 && K >= 4096;
#else
  const bool wgrad_big = false;
#endif
  pl.big = (!wgrad && t256 >= kCUs) || wgrad_big;
  const int64_t tiles = pl.big ? t256 : t128;
  pl.tiles = static_cast<int>(tiles);
  const int nkt = (hilo ? 3 : 1) * ((K + BK - 1) / BK);
  const int64_t want_wgs = !pl.big ? 2 * kCUs : kCUs;
  int splits = 1;
  // fp32 outputs and plain bf16 outputs (no epilogue or a bias, no hi/lo operands; a
  // stochastically rounded gradient among them) split K when the tiles leave CUs idle: partials
  // in fp32, then split_reduce_kernel (fp32) or split_reduce_bf16_kernel (bias added, rounded as
  // the unsplit epilogue would). Hi/lo bf16 products stay whole, equal to mg_gemm_hilo_prefix's
  // columns. 128 x 128 tiles aim at two workgroups per CU (measured at [1, 2048] chunks of the
  // d1024 expansion-3 model: 369 -> 351 ms per optimizer step against one; four: 378 ms).
  const bool split_ok = c_dtype == MG_F32 || (c_dtype == MG_BF16 && !hilo);
  const bool epi_ok = epilogue == MG_EPI_NONE || (epilogue == MG_EPI_BIAS && c_dtype == MG_BF16 && !hilo);
  if (epi_ok && split_ok && tiles < want_wgs && !deterministic)
    splits = static_cast<int>(std::min<int64_t>(std::max<int64_t>(want_wgs / tiles, 1), std::max(nkt / 4, 1)));
  pl.kt_per_split = std::max((nkt + splits - 1) / splits, 1);
  pl.ysplits = std::max((nkt + pl.kt_per_split - 1) / pl.kt_per_split, 1);
  return pl;
}

// Workspace of a split plan: the partials.
inline size_t ws_bytes(const Plan& pl, int M, int N) {
  if (pl.ysplits <= 1) return 0;
  return static_cast<size_t>(pl.ysplits) * M * N * sizeof(float);
}

template <int BM, int BN, int WM, int WN, bool AK, bool BKM, int EPI, typename TC, int CMODE>
int launch(const Params& p0, const Plan& pl, hipStream_t stream) {
  Params p = p0;
  p.tiles_m = (p.M + BM - 1) / BM;
  p.tiles_n = (p.N + BN - 1) / BN;
  p.kt_per_split = pl.kt_per_split;
  const int tiles = p.tiles_m * p.tiles_n;
  // K-split products run as a 1-D grid laid out by split_tile_of when it can
  // (MG_GEMM_XCD_SPLIT=0 in the environment turns that off)
  const char* e = getenv("MG_GEMM_XCD_SPLIT");
  if (CMODE == C_SPLIT && (tiles * pl.ysplits) % 8 == 0 && !(e && atoi(e) == 0)) {
    p.xcd_splits = pl.ysplits;
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, AK, BKM, EPI, TC, CMODE>), dim3(tiles * pl.ysplits), dim3(64 * WM * WN),
                       0, stream, p);
  } else {
    p.xcd_splits = 0;
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, AK, BKM, EPI, TC, CMODE>), dim3(tiles, pl.ysplits),
                       dim3(64 * WM * WN), 0, stream, p);
  }
  return check_launch("mg_gemm");
}

// The persistent kernel (gemm_persist_kernel): one workgroup per CU.
template <bool AK, bool BKM, int EPI>
int launch_persist(const Params& p0, hipStream_t stream) {
  Params p = p0;
  p.tiles_m = (p.M + 255) / 256;
  p.tiles_n = (p.N + 255) / 256;
  p.kt_per_split = total_ktiles(p);
  const int grid = std::min(p.tiles_m * p.tiles_n, kCUs);
  hipLaunchKernelGGL((gemm_persist_kernel<AK, BKM, EPI>), dim3(grid), dim3(512), 0, stream, p);
  return check_launch("mg_gemm");
}

// The persistent four-wave kernel (gemm_persist_w4m_kernel): one workgroup per CU.
template <bool AK, bool BKM, int EPI>
int launch_persist_w4m(const Params& p0, hipStream_t stream) {
  Params p = p0;
  p.tiles_m = (p.M + 255) / 256;
  p.tiles_n = (p.N + 255) / 256;
  p.kt_per_split = total_ktiles(p);
  const int grid = std::min(p.tiles_m * p.tiles_n, kCUs);
  hipLaunchKernelGGL((gemm_persist_w4m_kernel<AK, BKM, EPI>), dim3(grid), dim3(256), 0, stream, p);
  return check_launch("mg_gemm");
}

// Whether a product that meets the eight-wave loop's conditions runs
// persistent: a bf16 output written whole (no split, no accumulation), an
// epilogue done in registers, an even k-tile count, and more tiles than CUs.
// MG_GEMM_PERSIST=0 in the environment turns the persistent kernel off (read
// per call, so tests can compare both kernels in one process).
inline bool persist_ok(const Params& p, const Plan& pl, int epi, int c_dtype) {
  const char* e = getenv("MG_GEMM_PERSIST");
  const int mode = e ? atoi(e) : 1;
  if (!mode || c_dtype != MG_BF16 || pl.ysplits > 1 || p.accumulate) return false;
  if (epi != EPI_NONE && epi != EPI_BIAS && epi != EPI_BIAS_GELU && epi != EPI_SR) return false;
  if (total_ktiles(p) % 2) return false;
  const int64_t tiles = int64_t((p.M + 255) / 256) * ((p.N + 255) / 256);
  // the four-wave kernel's epilogue (in registers, no workgroup barrier) also
  // serves products of one tile per CU
  return tiles > kCUs || mode == 2 || (kUseW4M && mode != 3);
}

template <bool AK, bool BKM>
int dispatch_persist(const Params& p, int epi, hipStream_t s) {
  if constexpr (kUseW4M) {
    if (epi == EPI_NONE) return launch_persist_w4m<AK, BKM, EPI_NONE>(p, s);
    if (epi == EPI_BIAS) return launch_persist_w4m<AK, BKM, EPI_BIAS>(p, s);
    if (epi == EPI_BIAS_GELU) return launch_persist_w4m<AK, BKM, EPI_BIAS_GELU>(p, s);
    return launch_persist_w4m<AK, BKM, EPI_SR>(p, s);
  } else {
    if (epi == EPI_NONE) return launch_persist<AK, BKM, EPI_NONE>(p, s);
    if (epi == EPI_BIAS) return launch_persist<AK, BKM, EPI_BIAS>(p, s);
    if (epi == EPI_BIAS_GELU) return launch_persist<AK, BKM, EPI_BIAS_GELU>(p, s);
    return launch_persist<AK, BKM, EPI_SR>(p, s);
  }
}

template <int BM, int BN, int WM, int WN, bool AK, bool BKM>
int dispatch_epi(const Params& p, const Plan& pl, int epi, int c_dtype, hipStream_t s) {
  if (c_dtype == MG_F32) {
    if (pl.ysplits > 1) return launch<BM, BN, WM, WN, AK, BKM, EPI_NONE, float, C_SPLIT>(p, pl, s);
    if (p.accumulate) return launch<BM, BN, WM, WN, AK, BKM, EPI_NONE, float, C_ADD>(p, pl, s);
    if (epi == EPI_NONE) return launch<BM, BN, WM, WN, AK, BKM, EPI_NONE, float, C_STORE>(p, pl, s);
    if (epi == EPI_BIAS) return launch<BM, BN, WM, WN, AK, BKM, EPI_BIAS, float, C_STORE>(p, pl, s);
  } else {
    if (pl.ysplits > 1) return launch<BM, BN, WM, WN, AK, BKM, EPI_NONE, float, C_SPLIT>(p, pl, s);
    if (epi == EPI_NONE) return launch<BM, BN, WM, WN, AK, BKM, EPI_NONE, bf16_t, C_STORE>(p, pl, s);
    if (epi == EPI_BIAS) return launch<BM, BN, WM, WN, AK, BKM, EPI_BIAS, bf16_t, C_STORE>(p, pl, s);
    if (epi == EPI_BIAS_GELU) return launch<BM, BN, WM, WN, AK, BKM, EPI_BIAS_GELU, bf16_t, C_STORE>(p, pl, s);
    if constexpr (!(WM == 4 && WN == 2))  // (no room for the pre-activation staging next to eight waves)
      if (epi == EPI_GELU_GRAD) return launch<BM, BN, WM, WN, AK, BKM, EPI_GELU_GRAD, bf16_t, C_STORE>(p, pl, s);
    if (epi == EPI_SR) return launch<BM, BN, WM, WN, AK, BKM, EPI_SR, bf16_t, C_STORE>(p, pl, s);
  }
  return fail(MG_ERR_ARG, "mg_gemm: epilogue %d not available for this output dtype", epi);
}

// Whether a product meets the pipelined loops' no-mask conditions.
inline bool w4_ok(const Params& p, bool ak, bool bk) {
  if ((ak || bk) && p.K % BK) return false;
  if (!ak && p.M % kW4Rows) return false;
  if (!bk && p.N % kW4Rows) return false;
  return true;
}

// 256 x 256 tiles run the eight-wave pipelined loop (mainloop_w8) when the
// product meets the no-mask conditions (w4_ok); the GELU-gradient epilogue
// (whose pre-activation staging needs the second operand stage) runs the
// four-wave one (mainloop_w4); other products the masked 8-wave loops.
template <int BM, int BN>
int dispatch_layout(const Params& p, const Plan& pl, bool ak, bool bk, int epi, int c_dtype, hipStream_t s) {
  constexpr int WN = BM * BN >= 256 * 256 ? 4 : 2;
#ifndef MG_GEMM_NO_W4
  if constexpr (BM == 256 && BN == 256) {
#ifndef MG_GEMM_NO_W8
    if (w4_ok(p, ak, bk) && epi != EPI_GELU_GRAD) {
      if (persist_ok(p, pl, epi, c_dtype)) {
        if (ak && bk) return dispatch_persist<true, true>(p, epi, s);
        if (ak && !bk) return dispatch_persist<true, false>(p, epi, s);
        if (!ak && !bk) return dispatch_persist<false, false>(p, epi, s);
        return dispatch_persist<false, true>(p, epi, s);
      }
      // mainloop_w4m (2 x 2 waves), else mainloop_w8 (4 x 2)
      if (kUseW4M) {
        if (ak && bk) return dispatch_epi<256, 256, 2, 2, true, true>(p, pl, epi, c_dtype, s);
        if (ak && !bk) return dispatch_epi<256, 256, 2, 2, true, false>(p, pl, epi, c_dtype, s);
        if (!ak && !bk) return dispatch_epi<256, 256, 2, 2, false, false>(p, pl, epi, c_dtype, s);
        return dispatch_epi<256, 256, 2, 2, false, true>(p, pl, epi, c_dtype, s);
      }
      if (ak && bk) return dispatch_epi<256, 256, 4, 2, true, true>(p, pl, epi, c_dtype, s);
      if (ak && !bk) return dispatch_epi<256, 256, 4, 2, true, false>(p, pl, epi, c_dtype, s);
      if (!ak && !bk) return dispatch_epi<256, 256, 4, 2, false, false>(p, pl, epi, c_dtype, s);
      return dispatch_epi<256, 256, 4, 2, false, true>(p, pl, epi, c_dtype, s);
    }
#endif
    if (w4_ok(p, ak, bk)) {
      if (ak && bk) return dispatch_epi<256, 256, 2, 2, true, true>(p, pl, epi, c_dtype, s);
      if (ak && !bk) return dispatch_epi<256, 256, 2, 2, true, false>(p, pl, epi, c_dtype, s);
      if (!ak && !bk) return dispatch_epi<256, 256, 2, 2, false, false>(p, pl, epi, c_dtype, s);
      return dispatch_epi<256, 256, 2, 2, false, true>(p, pl, epi, c_dtype, s);
    }
  }
#endif
  if (ak && bk) return dispatch_epi<BM, BN, 2, WN, true, true>(p, pl, epi, c_dtype, s);
  if (ak && !bk) return dispatch_epi<BM, BN, 2, WN, true, false>(p, pl, epi, c_dtype, s);
  if (!ak && !bk) return dispatch_epi<BM, BN, 2, WN, false, false>(p, pl, epi, c_dtype, s);
  return dispatch_epi<BM, BN, 2, WN, false, true>(p, pl, epi, c_dtype, s);
}

// Split plan of a weight-gradient pair (both operands MN-contiguous, fp32
// outputs written or added, 256 x 256 tiles): the pair runs as one launch
// when each product has at least 16 tiles (as a lone weight gradient needs
// for 256 x 256 tiles), the two together fewer than one per CU, and a split
// count that keeps both XCD layouts whole. Otherwise each product runs alone.
struct PairPlan {
  bool ok;
  int t0, t1, kt_per_split, splits;
};

inline PairPlan pair_plan(int M0, int N0, int M1, int N1, int K, bool deterministic) {
  PairPlan pp{};
  if (deterministic || K < 1 || M0 % 256 || N0 % 256 || M1 % 256 || N1 % 256) return pp;
  pp.t0 = (M0 / 256) * (N0 / 256);
  pp.t1 = (M1 / 256) * (N1 / 256);
  if (pp.t0 < 16 || pp.t1 < 16 || pp.t0 + pp.t1 >= kCUs) return pp;
  const int nkt = (K + BK - 1) / BK;
  const int want = std::min(std::max(kCUs / (pp.t0 + pp.t1), 1), std::max(nkt / 4, 1));
  pp.kt_per_split = (nkt + want - 1) / want;
  pp.splits = (nkt + pp.kt_per_split - 1) / pp.kt_per_split;
  pp.ok = pp.splits >= 2 && (pp.t0 * pp.splits) % 8 == 0 && (pp.t1 * pp.splits) % 8 == 0;
  return pp;
}

inline int launch_pair(Params p0, Params p1, const PairPlan& pp, hipStream_t s) {
  for (Params* p : {&p0, &p1}) {
    p->tiles_m = p->M / 256;
    p->tiles_n = p->N / 256;
    p->kt_per_split = pp.kt_per_split;
    p->xcd_splits = pp.splits;
  }
  constexpr int kWM = kUseW4M ? 2 : 4;  // mainloop_w4m (2 x 2 waves) or mainloop_w8 (4 x 2)
  hipLaunchKernelGGL((gemm_pair_kernel<256, 256, kWM, 2, false, false>), dim3((pp.t0 + pp.t1) * pp.splits),
                     dim3(64 * kWM * 2), 0, s, p0, p1, pp.t0 * pp.splits);
  if (check_launch("mg_gemm_wgrad_pair")) return MG_ERR_HIP;
  for (const Params* p : {&p0, &p1}) {
    const int64_t n4 = int64_t(p->M) * (p->N / 4);
    hipLaunchKernelGGL(split_reduce_kernel, dim3(static_cast<int>(std::min<int64_t>((n4 + 255) / 256, 2048))), dim3(256),
                       0, s, p->part, pp.splits, p->M, p->N, static_cast<float*>(p->C), p->ldc, p->accumulate);
  }
  return check_launch("mg_gemm_wgrad_pair");
}

}  // namespace gemm
}  // namespace mg

using namespace mg;

extern "C" int mg_gemm(int a_layout, const void* A, int64_t lda, int b_layout, const void* B, int64_t ldb, int M,
                       int N, int K, int epilogue, const float* bias, void* aux, int64_t ldaux, int c_dtype, void* C,
                       int64_t ldc, int flags, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "mg_gemm";
  if (flags & ~(MG_GEMM_ACCUMULATE | MG_GEMM_DETERMINISTIC | MG_GEMM_HILO | MG_GEMM_STOCHASTIC))
    return fail(MG_ERR_ARG, "%s: unknown flags %d", fn, flags);
  if ((flags & MG_GEMM_STOCHASTIC) && (c_dtype != MG_BF16 || (epilogue != MG_EPI_NONE && epilogue != MG_EPI_GELU_GRAD)))
    return fail(MG_ERR_ARG, "%s: stochastic rounding needs a bf16 C and no epilogue (or the GELU gradient's)", fn);
  const bool accumulate = flags & MG_GEMM_ACCUMULATE;
  const bool deterministic = flags & MG_GEMM_DETERMINISTIC;
  const bool hilo = flags & MG_GEMM_HILO;
  if (!A || !B || !C) return fail(MG_ERR_ARG, "%s: null operand", fn);
  if (M < 0 || N < 0 || K < 0) return fail(MG_ERR_ARG, "%s: negative size", fn);
  if ((a_layout != MG_KCONTIG && a_layout != MG_MNCONTIG) || (b_layout != MG_KCONTIG && b_layout != MG_MNCONTIG))
    return fail(MG_ERR_ARG, "%s: bad layout code", fn);
  if (c_dtype != MG_F32 && c_dtype != MG_BF16) return fail(MG_ERR_DTYPE, "%s: bad output dtype %d", fn, c_dtype);
  if (epilogue < MG_EPI_NONE || epilogue > MG_EPI_GELU_GRAD) return fail(MG_ERR_ARG, "%s: bad epilogue %d", fn, epilogue);
  if (N % 8) return fail(MG_ERR_ARG, "%s: N (%d) must be a multiple of 8", fn, N);
  if ((a_layout == MG_KCONTIG || b_layout == MG_KCONTIG) && K % 8)
    return fail(MG_ERR_ARG, "%s: K (%d) must be a multiple of 8 for a K-contiguous operand", fn, K);
  if (a_layout == MG_MNCONTIG && M % 8) return fail(MG_ERR_ARG, "%s: M (%d) must be a multiple of 8 for an MN-contiguous A", fn, M);
  if (lda % 8 || ldb % 8 || ldc % (c_dtype == MG_F32 ? 4 : 8) || (aux && ldaux % 8))
    return fail(MG_ERR_ARG, "%s: leading dimensions must span whole 16-byte chunks", fn);
  if (!aligned(A, 16) || !aligned(B, 16) || !aligned(C, 16) || (aux && !aligned(aux, 16)) || (bias && !aligned(bias, 16)))
    return fail(MG_ERR_ARG, "%s: operands must be 16-byte aligned", fn);
  if (hilo && (a_layout != MG_KCONTIG || b_layout != MG_KCONTIG || K < 1))
    return fail(MG_ERR_ARG, "%s: hi/lo products need K-contiguous A and B and K >= 1", fn);
  const int krow = hilo ? 2 * K : K;  // elements of a K-contiguous row
  if (lda < (a_layout == MG_KCONTIG ? krow : M) || ldb < (b_layout == MG_KCONTIG ? krow : N) || ldc < N)
    return fail(MG_ERR_ARG, "%s: leading dimension smaller than the row", fn);
  if ((epilogue == MG_EPI_BIAS || epilogue == MG_EPI_BIAS_GELU) && !bias)
    return fail(MG_ERR_ARG, "%s: epilogue needs bias", fn);
  if ((epilogue == MG_EPI_BIAS_GELU || epilogue == MG_EPI_GELU_GRAD) && (!aux || ldaux < N || c_dtype != MG_BF16))
    return fail(MG_ERR_ARG, "%s: GELU epilogues need aux (bf16, ldaux >= N) and a bf16 output", fn);
  if (accumulate && (c_dtype != MG_F32 || epilogue != MG_EPI_NONE))
    return fail(MG_ERR_ARG, "%s: accumulate needs an fp32 output and no epilogue", fn);
  if (M == 0 || N == 0) return MG_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);

  gemm::Params p{};
  p.A = static_cast<const bf16_t*>(A);
  p.B = static_cast<const bf16_t*>(B);
  p.C = C;
  p.bias = bias;
  p.aux = static_cast<bf16_t*>(aux);
  p.lda = lda; p.ldb = ldb; p.ldc = ldc; p.ldaux = ldaux;
  p.M = M; p.N = N; p.K = K;
  const bool ak = a_layout == MG_KCONTIG, bk = b_layout == MG_KCONTIG;
  // bytes spanned by each operand; buffer offsets are 32-bit
  const int64_t a_span = ak ? (int64_t(M - 1) * lda + krow) * 2 : (int64_t(std::max(K, 1) - 1) * lda + M) * 2;
  const int64_t b_span = bk ? (int64_t(N - 1) * ldb + krow) * 2 : (int64_t(std::max(K, 1) - 1) * ldb + N) * 2;
  if (a_span + 256 * lda * 2 >= (int64_t(1) << 31) || b_span + 256 * ldb * 2 >= (int64_t(1) << 31))
    return fail(MG_ERR_ARG, "%s: operands must span less than 2 GiB", fn);
  p.a_span = static_cast<uint32_t>(a_span);
  p.b_span = static_cast<uint32_t>(b_span);
  if (aux) {
    const int64_t aux_span = (int64_t(M - 1) * ldaux + N) * 2;
    if (aux_span + 256 * ldaux * 2 >= (int64_t(1) << 31)) return fail(MG_ERR_ARG, "%s: aux must span less than 2 GiB", fn);
    p.aux_span = static_cast<uint32_t>(aux_span);
  }

  p.hilo = hilo ? 1 : 0;
  p.nkt_seg = (K + gemm::BK - 1) / gemm::BK;
  if (K == 0 && accumulate) return MG_OK;
  // Without a workspace the product runs unsplit.
  gemm::Plan pl = gemm::plan(M, N, K, ak, bk, c_dtype, epilogue, deterministic || !workspace, hilo);
  if (pl.ysplits > 1) {
    const size_t need = gemm::ws_bytes(pl, M, N);
    if (workspace_bytes < need)
      return fail(MG_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu (mg_gemm_workspace_bytes)", fn,
                  workspace_bytes, need);
    if (!aligned(workspace, 16)) return fail(MG_ERR_ARG, "%s: workspace not 16-byte aligned", fn);
    p.part = static_cast<float*>(workspace);
  }
  p.accumulate = accumulate ? 1 : 0;
  const int epi = (flags & MG_GEMM_STOCHASTIC) && epilogue == MG_EPI_NONE ? gemm::EPI_SR : epilogue;
  const int rc = pl.big ? gemm::dispatch_layout<256, 256>(p, pl, ak, bk, epi, c_dtype, s)
                        : gemm::dispatch_layout<128, 128>(p, pl, ak, bk, epi, c_dtype, s);
  if (rc || pl.ysplits <= 1) return rc;
  const int64_t n4 = int64_t(M) * (N / 4);
  const dim3 rgrid(static_cast<int>(std::min<int64_t>((n4 + 255) / 256, 2048)));
  if (c_dtype == MG_F32)
    hipLaunchKernelGGL(gemm::split_reduce_kernel, rgrid, dim3(256), 0, s, p.part, pl.ysplits, M, N,
                       static_cast<float*>(C), ldc, p.accumulate);
  else
    hipLaunchKernelGGL(gemm::split_reduce_bf16_kernel, rgrid, dim3(256), 0, s, p.part, pl.ysplits, M, N,
                       static_cast<bf16_t*>(C), ldc, (flags & MG_GEMM_STOCHASTIC) ? 1 : 0,
                       epilogue == MG_EPI_BIAS ? bias : nullptr);
  return check_launch(fn);
}

extern "C" int mg_gemm_hilo_prefix(const void* A, int64_t lda, const void* B, int64_t ldb, int M, int N, int K,
                                   int hilo_cols, void* C, int64_t ldc, void* stream) {
  const char* fn = "mg_gemm_hilo_prefix";
  if (!A || !B || !C) return fail(MG_ERR_ARG, "%s: null operand", fn);
  if (!gemm::kUseW4M) return fail(MG_ERR_ARG, "%s: needs the four-wave persistent kernel", fn);
  if (M < 1 || N < 8 || N % 8 || K < 64 || K % 128)
    return fail(MG_ERR_ARG, "%s: M=%d N=%d K=%d (N a multiple of 8, K of 128)", fn, M, N, K);
  if (hilo_cols < 256 || hilo_cols % 256 || hilo_cols >= N)
    return fail(MG_ERR_ARG, "%s: hilo_cols %d must be a multiple of 256 below N=%d", fn, hilo_cols, N);
  if (lda < 2 * K || ldb < 2 * K || ldc < N || lda % 8 || ldb % 8 || ldc % 8)
    return fail(MG_ERR_ARG, "%s: leading dimensions (rows of 2K hi/lo values, ldc >= N, multiples of 8)", fn);
  if (!aligned(A, 16) || !aligned(B, 16) || !aligned(C, 16)) return fail(MG_ERR_ARG, "%s: operands must be 16-byte aligned", fn);
  const int64_t a_span = (int64_t(M - 1) * lda + 2 * K) * 2, b_span = (int64_t(N - 1) * ldb + 2 * K) * 2;
  if (a_span + 256 * lda * 2 >= (int64_t(1) << 31) || b_span + 256 * ldb * 2 >= (int64_t(1) << 31))
    return fail(MG_ERR_ARG, "%s: operands must span less than 2 GiB", fn);
  gemm::Params p{};
  p.A = static_cast<const bf16_t*>(A);
  p.B = static_cast<const bf16_t*>(B);
  p.C = C;
  p.lda = lda; p.ldb = ldb; p.ldc = ldc;
  p.M = M; p.N = N; p.K = K;
  p.a_span = static_cast<uint32_t>(a_span);
  p.b_span = static_cast<uint32_t>(b_span);
  p.hilo = 1;
  p.nkt_seg = K / gemm::BK;  // even: K % 128 == 0
  p.hilo_cols = hilo_cols;
  p.tiles_m = (M + 255) / 256;
  p.tiles_n = (N + 255) / 256;
  p.kt_per_split = 3 * p.nkt_seg;
  hipLaunchKernelGGL((gemm::gemm_persist_w4m_kernel<true, true, gemm::EPI_NONE, true>),
                     dim3(std::min(p.tiles_m * p.tiles_n, gemm::kCUs)), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  return check_launch(fn);
}

extern "C" size_t mg_gemm_workspace_bytes(int a_layout, int b_layout, int M, int N, int K, int epilogue,
                                          int c_dtype, int flags) {
  if (M < 1 || N < 1 || K < 1) return 0;
  const gemm::Plan pl = gemm::plan(M, N, K, a_layout == MG_KCONTIG, b_layout == MG_KCONTIG, c_dtype, epilogue,
                                   flags & MG_GEMM_DETERMINISTIC, flags & MG_GEMM_HILO);
  return gemm::ws_bytes(pl, M, N);
}

extern "C" size_t mg_gemm_wgrad_pair_workspace_bytes(int M0, int N0, int M1, int N1, int K, int flags) {
  if (M0 < 1 || N0 < 1 || M1 < 1 || N1 < 1 || K < 1) return 0;
  const gemm::PairPlan pp = gemm::pair_plan(M0, N0, M1, N1, K, flags & MG_GEMM_DETERMINISTIC);
  if (pp.ok) return static_cast<size_t>(pp.splits) * (size_t(M0) * N0 + size_t(M1) * N1) * sizeof(float);
  return std::max(mg_gemm_workspace_bytes(MG_MNCONTIG, MG_MNCONTIG, M0, N0, K, MG_EPI_NONE, MG_F32, flags),
                  mg_gemm_workspace_bytes(MG_MNCONTIG, MG_MNCONTIG, M1, N1, K, MG_EPI_NONE, MG_F32, flags));
}

extern "C" int mg_gemm_wgrad_pair(const void* dy0, int64_t ld_dy0, const void* x0, int64_t ld_x0, int M0, int N0,
                                  float* dw0, int64_t ldc0, const void* dy1, int64_t ld_dy1, const void* x1,
                                  int64_t ld_x1, int M1, int N1, float* dw1, int64_t ldc1, int K, int flags,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "mg_gemm_wgrad_pair";
  if (flags & ~(MG_GEMM_ACCUMULATE | MG_GEMM_DETERMINISTIC)) return fail(MG_ERR_ARG, "%s: unknown flags %d", fn, flags);
  if (!dy0 || !x0 || !dw0 || !dy1 || !x1 || !dw1) return fail(MG_ERR_ARG, "%s: null operand", fn);
  if (M0 < 0 || N0 < 0 || M1 < 0 || N1 < 0 || K < 0) return fail(MG_ERR_ARG, "%s: negative size", fn);
  const gemm::PairPlan pp = gemm::pair_plan(M0, N0, M1, N1, K, (flags & MG_GEMM_DETERMINISTIC) || !workspace);
  if (!pp.ok) {  // each product alone (mg_gemm validates its arguments)
    int rc = mg_gemm(MG_MNCONTIG, dy0, ld_dy0, MG_MNCONTIG, x0, ld_x0, M0, N0, K, MG_EPI_NONE, nullptr, nullptr, 0, MG_F32,
                     dw0, ldc0, flags, workspace, workspace_bytes, stream);
    if (rc) return rc;
    return mg_gemm(MG_MNCONTIG, dy1, ld_dy1, MG_MNCONTIG, x1, ld_x1, M1, N1, K, MG_EPI_NONE, nullptr, nullptr, 0, MG_F32,
                   dw1, ldc1, flags, workspace, workspace_bytes, stream);
  }
  // (pp.ok: M and N are positive multiples of 256, K >= 1)
  const void* A[2] = {dy0, dy1};
  const void* B[2] = {x0, x1};
  float* C[2] = {dw0, dw1};
  const int64_t lda[2] = {ld_dy0, ld_dy1}, ldb[2] = {ld_x0, ld_x1}, ldc[2] = {ldc0, ldc1};
  const int Ms[2] = {M0, M1}, Ns[2] = {N0, N1};
  gemm::Params p[2] = {};
  const size_t need = static_cast<size_t>(pp.splits) * (size_t(M0) * N0 + size_t(M1) * N1) * sizeof(float);
  if (workspace_bytes < need)
    return fail(MG_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu (mg_gemm_wgrad_pair_workspace_bytes)", fn,
                workspace_bytes, need);
  if (!aligned(workspace, 16)) return fail(MG_ERR_ARG, "%s: workspace not 16-byte aligned", fn);
  float* part = static_cast<float*>(workspace);
  for (int i = 0; i < 2; ++i) {
    const int M = Ms[i], N = Ns[i];
    if (lda[i] % 8 || ldb[i] % 8 || ldc[i] % 4) return fail(MG_ERR_ARG, "%s: leading dimensions must span whole 16-byte chunks", fn);
    if (lda[i] < M || ldb[i] < N || ldc[i] < N) return fail(MG_ERR_ARG, "%s: leading dimension smaller than the row", fn);
    if (!aligned(A[i], 16) || !aligned(B[i], 16) || !aligned(C[i], 16))
      return fail(MG_ERR_ARG, "%s: operands must be 16-byte aligned", fn);
    const int64_t a_span = (int64_t(K - 1) * lda[i] + M) * 2, b_span = (int64_t(K - 1) * ldb[i] + N) * 2;
    if (a_span + 256 * lda[i] * 2 >= (int64_t(1) << 31) || b_span + 256 * ldb[i] * 2 >= (int64_t(1) << 31))
      return fail(MG_ERR_ARG, "%s: operands must span less than 2 GiB", fn);
    gemm::Params& q = p[i];
    q.A = static_cast<const bf16_t*>(A[i]);
    q.B = static_cast<const bf16_t*>(B[i]);
    q.C = C[i];
    q.lda = lda[i]; q.ldb = ldb[i]; q.ldc = ldc[i];
    q.M = M; q.N = N; q.K = K;
    q.a_span = static_cast<uint32_t>(a_span);
    q.b_span = static_cast<uint32_t>(b_span);
    q.nkt_seg = (K + gemm::BK - 1) / gemm::BK;
    q.accumulate = (flags & MG_GEMM_ACCUMULATE) ? 1 : 0;
    q.part = part;
    part += static_cast<size_t>(pp.splits) * M * N;
  }
  return gemm::launch_pair(p[0], p[1], pp, static_cast<hipStream_t>(stream));
}

extern "C" int mg_logits_cross_entropy_partials(int64_t N) {
  return N < 1 ? 0 : static_cast<int>((N + gemm::kCeRows - 1) / gemm::kCeRows);
}

extern "C" int mg_logits_cross_entropy(const void* embed, int64_t lde, const void* w, int64_t ldw,
                                       const int64_t* labels, void* dlogits, int64_t ldd, float* loss_part,
                                       int* bad_label, int N, int D, int V, float scale, void* stream) {
  const char* fn = "mg_logits_cross_entropy";
  if (!embed || !w || !labels || !dlogits || !loss_part) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (N < 1 || D < 8 || D % 8 || V < 8 || V > 256 || V % 8)
    return fail(MG_ERR_ARG, "%s: bad shape N=%d D=%d V=%d (D %% 8 == 0, 8 <= V <= 256, V %% 8 == 0)", fn, N, D, V);
  if (lde < D || lde % 8 || ldw < D || ldw % 8 || ldd < V || ldd % 4)
    return fail(MG_ERR_ARG, "%s: bad leading dimensions", fn);
  if (!aligned(embed, 16) || !aligned(w, 16) || !aligned(dlogits, 8) || !aligned(labels, 8))
    return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  const int64_t a_span = (int64_t(N - 1) * lde + D) * 2, b_span = (int64_t(V - 1) * ldw + D) * 2;
  if (a_span + 256 * lde * 2 >= (int64_t(1) << 31)) return fail(MG_ERR_ARG, "%s: embed spans 2 GiB or more", fn);
  gemm::Params p{};
  p.A = static_cast<const bf16_t*>(embed);
  p.B = static_cast<const bf16_t*>(w);
  p.lda = lde; p.ldb = ldw;
  p.M = N; p.N = V; p.K = D;
  p.a_span = static_cast<uint32_t>(a_span);
  p.b_span = static_cast<uint32_t>(b_span);
  hipLaunchKernelGGL(gemm::logits_ce_kernel, dim3((N + gemm::kCeRows - 1) / gemm::kCeRows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p, labels, static_cast<bf16_t*>(dlogits), ldd, loss_part,
                     bad_label, scale);
  return check_launch(fn);
}
