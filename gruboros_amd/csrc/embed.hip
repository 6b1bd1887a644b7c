// Token-embedding weight gradient (reference mingru/minLM.py:92,99: nn.Embedding,
// whose backward adds each row of the output gradient into the weight row of
// its token id):
//
//   dw[v, :] = sum over tokens t with ids[t] == v of dx[t, :]     (fp32)
//
// torch's version sorts the ids and sizes its segment buffers from a count it
// copies to the host, so the host stops there until the GPU has caught up, at
// the end of every backward pass, and the optimizer's host work then runs with
// the GPU idle. This one is three launches with no host round trip, and it sums
// in a fixed order (token order within a chunk, chunks in order), so results
// repeat bit for bit:
//   1. embed_sort_kernel (one workgroup): a stable counting sort of the ids.
//      perm lists the token indices grouped by id, in token order; off[v] is
//      the first position of id v; cst[v] its first chunk, chunks being runs
//      of up to kChunk positions of one id (a frequent id gets many chunks, so
//      no workgroup of step 2 sums more than kChunk rows).
//   2. embed_chunk_kernel: workgroup b sums the dx rows of chunk b, in order,
//      into part[b, :].
//   3. embed_reduce_kernel: dw[v, :] = the sum of id v's chunk rows, in chunk
//      order (zero for an id with no token).
// Ids outside [0, V) are skipped: the forward gather has already refused them.

#include <algorithm>

#include "mg_common.h"

namespace mg {
namespace embed {

constexpr int kSortWaves = 16;                 // waves of the sorting workgroup
constexpr int kMaxV = 512;                     // ids fit 9 bits
constexpr int kIdBits = 9;
constexpr int kChunk = 64;                     // positions per chunk
constexpr int kThreads = 256;                  // chunk / reduce workgroups: 4 columns per thread
constexpr int kCols = kThreads * 4;

inline int64_t max_chunks(int64_t N, int V) { return (N + kChunk - 1) / kChunk + V; }

// Lanes of this wave holding the same id as this lane (v >= 0), from one
// ballot per id bit.
__device__ __forceinline__ uint64_t peers_of(int v) {
  uint64_t m = __ballot(v >= 0);
#pragma unroll
  for (int b = 0; b < kIdBits; ++b) {
    const uint64_t bb = __ballot(v >= 0 && ((v >> b) & 1));
    m &= ((v >> b) & 1) ? bb : ~bb;
  }
  return m;
}

// Wave w walks tokens [w per, (w + 1) per) 64 at a time, kBatch rounds per
// batch of loads (a batch's ids are loaded before its first round, so a wave
// waits for memory once per batch, not once per round). Per round, a lane's
// rank among the round's lanes of its id comes from the peer mask; run[v]
// counts the wave's tokens of id v so far (read by every lane of the group,
// then advanced by the group's last lane: a wave's LDS accesses run in
// program order). `emit` gets (token, id, run + rank).
constexpr int kBatch = 16;
template <typename F>
__device__ __forceinline__ void walk(const int64_t* __restrict__ ids, int64_t t0, int64_t t1, int V, int* run,
                                     F&& emit) {
  const int lane = threadIdx.x & 63;
  for (int64_t base = t0; base < t1; base += 64 * kBatch) {
    int vs[kBatch];
#pragma unroll
    for (int r = 0; r < kBatch; ++r) {
      const int64_t t = base + r * 64 + lane;
      const int64_t x = t < t1 ? ids[t] : -1;
      vs[r] = (x >= 0 && x < V) ? static_cast<int>(x) : -1;
    }
#pragma unroll
    for (int r = 0; r < kBatch; ++r) {
      const int v = vs[r];
      const uint64_t m = peers_of(v);
      if (v >= 0) {
        const int rk = __popcll(m & ((1ull << lane) - 1ull));
        const int c = run[v];
        emit(base + r * 64 + lane, v, c + rk);
        if (63 - __clzll(m) == lane) run[v] = c + __popcll(m);
      }
    }
  }
}

__global__ __launch_bounds__(kSortWaves * 64) void embed_sort_kernel(const int64_t* __restrict__ ids, int64_t N,
                                                                    int V, int* __restrict__ perm,
                                                                    int* __restrict__ off, int* __restrict__ cst) {
  __shared__ int cnt[kSortWaves][kMaxV];
  __shared__ int s_off[kMaxV + 1], s_cst[kMaxV + 1];
  const int wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kSortWaves * kMaxV; i += blockDim.x) (&cnt[0][0])[i] = 0;
  __syncthreads();
  const int64_t per = (N + kSortWaves - 1) / kSortWaves;
  const int64_t t0 = std::min<int64_t>(N, wave * per), t1 = std::min<int64_t>(N, t0 + per);
  // pass 1: each wave's count per id
  walk(ids, t0, t1, V, cnt[wave], [](int64_t, int, int) {});
  __syncthreads();
  // per id: the waves' counts become their exclusive prefix (wave w's first
  // position within the id), tot the id's count
  const int v = threadIdx.x;
  int tot = 0;
  if (v < V) {
    for (int w = 0; w < kSortWaves; ++w) {
      const int c = cnt[w][v];
      cnt[w][v] = tot;
      tot += c;
    }
  }
  // exclusive scans over the ids of the counts and of the chunk counts
  // (Hillis-Steele in LDS, ids 0 .. kMaxV - 1; ids past V count zero)
  const bool in = v < kMaxV;
  if (in) {
    s_off[v] = v < V ? tot : 0;
    s_cst[v] = v < V ? (tot + kChunk - 1) / kChunk : 0;
  }
  __syncthreads();
  for (int d = 1; d < kMaxV; d <<= 1) {
    int a = 0, b = 0;
    if (in && v >= d) {
      a = s_off[v - d];
      b = s_cst[v - d];
    }
    __syncthreads();
    if (in && v >= d) {
      s_off[v] += a;
      s_cst[v] += b;
    }
    __syncthreads();
  }
  // inclusive -> exclusive, published for steps 2 and 3
  if (v <= V) {
    off[v] = v == 0 ? 0 : s_off[v - 1];
    cst[v] = v == 0 ? 0 : s_cst[v - 1];
  }
  __syncthreads();
  // pass 2: positions (the counters restart from each wave's prefix)
  walk(ids, t0, t1, V, cnt[wave], [&](int64_t t, int id, int r) {
    const int pos = (id == 0 ? 0 : s_off[id - 1]) + r;
    perm[pos] = static_cast<int>(t);
  });
}

// part[b, :] = sum of dx over chunk b's tokens, in order.
__global__ __launch_bounds__(kThreads) void embed_chunk_kernel(const float* __restrict__ dx, int64_t ldx, int D,
                                                               int V, const int* __restrict__ perm,
                                                               const int* __restrict__ off,
                                                               const int* __restrict__ cst,
                                                               float* __restrict__ part) {
  __shared__ int s_t[kChunk];
  const int b = blockIdx.x;
  if (b >= cst[V]) return;
  // the id whose chunks include b: the largest v with cst[v] <= b (ids with
  // no token share their successor's cst and sort before it)
  int lo = 0, hi = V;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cst[mid] <= b) lo = mid;
    else hi = mid;
  }
  const int p0 = off[lo] + (b - cst[lo]) * kChunk;
  const int n = std::min(kChunk, off[lo + 1] - p0);
  if (threadIdx.x < n) s_t[threadIdx.x] = perm[p0 + threadIdx.x];
  __syncthreads();
  for (int c = threadIdx.x * 4; c < D; c += kCols) {
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int i = 0;
    for (; i + 8 <= n; i += 8) {  // eight rows in flight
      float4 r[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) r[u] = *reinterpret_cast<const float4*>(dx + s_t[i + u] * ldx + c);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        acc.x += r[u].x; acc.y += r[u].y; acc.z += r[u].z; acc.w += r[u].w;
      }
    }
    for (; i < n; ++i) {
      const float4 r = *reinterpret_cast<const float4*>(dx + s_t[i] * ldx + c);
      acc.x += r.x; acc.y += r.y; acc.z += r.z; acc.w += r.w;
    }
    *reinterpret_cast<float4*>(part + static_cast<int64_t>(b) * D + c) = acc;
  }
}

// dw[v, :] = sum of id v's chunk rows, in chunk order.
__global__ __launch_bounds__(kThreads) void embed_reduce_kernel(const float* __restrict__ part, int D,
                                                                const int* __restrict__ cst, float* __restrict__ dw,
                                                                int64_t ldw) {
  const int v = blockIdx.x;
  const int b0 = cst[v], b1 = cst[v + 1];
  for (int c = threadIdx.x * 4; c < D; c += kCols) {
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int b = b0; b < b1; ++b) {
      const float4 r = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(b) * D + c);
      acc.x += r.x; acc.y += r.y; acc.z += r.z; acc.w += r.w;
    }
    *reinterpret_cast<float4*>(dw + v * ldw + c) = acc;
  }
}

// Workspace: part [max_chunks][D] fp32, then perm [N], off [V + 1], cst [V + 1] int32.
inline size_t part_bytes(int64_t N, int D, int V) {
  return (static_cast<size_t>(max_chunks(N, V)) * D * sizeof(float) + 255) & ~size_t(255);
}

}  // namespace embed
}  // namespace mg

using namespace mg;

extern "C" size_t mg_embedding_bwd_workspace_bytes(int64_t N, int D, int V) {
  if (N < 1 || D < 1 || V < 1) return 16;
  return embed::part_bytes(N, D, V) + static_cast<size_t>(N + 2 * (V + 1)) * sizeof(int);
}

extern "C" int mg_embedding_bwd(const int64_t* ids, const float* dx, int64_t ldx, int64_t N, int D, int V, float* dw,
                                int64_t ldw, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "mg_embedding_bwd";
  if (!ids || !dx || !dw) return fail(MG_ERR_ARG, "%s: NULL pointer", fn);
  if (N < 1 || N >= (int64_t(1) << 31) || D < 4 || D % 4 || V < 1 || V > embed::kMaxV || ldx < D || ldx % 4 ||
      ldw < D || ldw % 4)
    return fail(MG_ERR_ARG, "%s: bad shape N=%lld D=%d V=%d ldx=%lld ldw=%lld (1 <= V <= %d, D and strides %% 4 == 0)",
                fn, (long long)N, D, V, (long long)ldx, (long long)ldw, embed::kMaxV);
  if (static_cast<int64_t>(N - 1) * ldx + D > (int64_t(1) << 31) || static_cast<int64_t>(V) * ldw > (int64_t(1) << 31))
    return fail(MG_ERR_ARG, "%s: dx or dw past 2^31 elements", fn);
  if (!aligned(dx, 16) || !aligned(dw, 16) || !aligned(ids, 8)) return fail(MG_ERR_ARG, "%s: misaligned pointer", fn);
  if (!workspace || workspace_bytes < mg_embedding_bwd_workspace_bytes(N, D, V) || !aligned(workspace, 16))
    return fail(MG_ERR_WORKSPACE, "%s: workspace too small or misaligned", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  int* perm = reinterpret_cast<int*>(static_cast<char*>(workspace) + embed::part_bytes(N, D, V));
  int* off = perm + N;
  int* cst = off + (V + 1);
  hipLaunchKernelGGL(embed::embed_sort_kernel, dim3(1), dim3(embed::kSortWaves * 64), 0, st, ids, N, V, perm, off,
                     cst);
  hipLaunchKernelGGL(embed::embed_chunk_kernel, dim3(static_cast<unsigned>(embed::max_chunks(N, V))),
                     dim3(embed::kThreads), 0, st, dx, ldx, D, V, perm, off, cst, part);
  hipLaunchKernelGGL(embed::embed_reduce_kernel, dim3(V), dim3(embed::kThreads), 0, st, part, D, cst, dw, ldw);
  return check_launch(fn);
}
