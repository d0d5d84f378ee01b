// Dispatch: per-expert histogram, exclusive prefix sum and a stable
// permutation of (token, slot) assignments into expert-major order, tokens
// ascending within an expert.
//
// Reference: Decoder::experts pushes (row, p) onto assignments[expert] while
// walking rows in order (src/decoder/mod.rs:127-141) and then visits experts
// in ascending id (:198-218); the permutation below is that order.
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {

int max_tiles(int T, int K, int E, int bm) {
  // Routed: sum_e ceil(n_e / bm) <= min(E, T*K) + T*K / bm. Shared: ceil(T / bm).
  long long tk = (long long)T * K;
  long long routed = (tk < E ? tk : E) + tk / bm;
  return (int)(routed + (T + bm - 1) / bm);
}

constexpr int kDispatchThreads = 1024;
constexpr int kDispatchWaves = kDispatchThreads / 64;

// One workgroup. Tokens are taken 1024 at a time (one per thread); inside a
// wave the rank of a token among earlier tokens of the same expert comes
// from a ballot, across waves from an LDS prefix, across chunks from a
// running count — together the stable counting sort.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(
    const int* __restrict__ ids, const float* __restrict__ w, int T, int E, int K, int bm,
    int* __restrict__ offsets, int* __restrict__ perm_rows, float* __restrict__ perm_w,
    int* __restrict__ inv_pos, int* __restrict__ tiles, int* __restrict__ counters) {
  __shared__ int count[64];
  __shared__ int base[64];
  __shared__ int running[64];
  __shared__ int chunk_total[64];
  __shared__ int wave_count[kDispatchWaves][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (tid < 64) {
    count[tid] = 0;
    running[tid] = 0;
  }
  __syncthreads();
  for (int i = tid; i < T * K; i += kDispatchThreads) atomicAdd(&count[ids[i]], 1);
  __syncthreads();
  if (wave == 0) {
    // Exclusive scan over experts (E <= 64 lanes).
    int c = lane < E ? count[lane] : 0;
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    int excl = incl - c;
    if (lane < E) {
      base[lane] = excl;
      offsets[lane] = excl;
    }
    if (lane == 0) offsets[E] = T * K;
    // Row tiles of bm rows per expert, then the shared expert's tiles.
    int nt = lane < E ? (c + bm - 1) / bm : 0;
    int tincl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int v = __shfl_up(tincl, o);
      if (lane >= o) tincl += v;
    }
    int tstart = tincl - nt;
    for (int i = 0; i < nt; i++) {
      tiles[2 * (tstart + i)] = lane;
      tiles[2 * (tstart + i) + 1] = i * bm;
    }
    int routed_tiles = __shfl(tincl, 63);
    int shared_tiles = (T + bm - 1) / bm;
    for (int i = lane; i < shared_tiles; i += 64) {
      tiles[2 * (routed_tiles + i)] = E;
      tiles[2 * (routed_tiles + i) + 1] = i * bm;
    }
    if (lane == 0) {
      counters[0] = routed_tiles + shared_tiles;
      counters[1] = routed_tiles;
    }
  }
  __syncthreads();
  for (int c0 = 0; c0 < T; c0 += kDispatchThreads) {
    const int t = c0 + tid;
    const bool valid = t < T;
    int my_e[8];
    int my_rank[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      my_e[j] = (valid && j < K) ? ids[(size_t)t * K + j] : -1;
      my_rank[j] = 0;
    }
    const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int e = 0; e < E; e++) {
      bool has = false;
#pragma unroll
      for (int j = 0; j < 8; j++) has |= my_e[j] == e;
      unsigned long long mask = __ballot(has);
      if (lane == 0) wave_count[wave][e] = __popcll(mask);
      int r = __popcll(mask & lt);
#pragma unroll
      for (int j = 0; j < 8; j++)
        if (my_e[j] == e) my_rank[j] = r;
    }
    __syncthreads();
    if (tid < E) {
      int acc = 0;
      for (int v = 0; v < kDispatchWaves; v++) {
        int c = wave_count[v][tid];
        wave_count[v][tid] = acc;
        acc += c;
      }
      chunk_total[tid] = acc;
    }
    __syncthreads();
    if (valid) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        if (j < K) {
          int e = my_e[j];
          int pos = base[e] + running[e] + wave_count[wave][e] + my_rank[j];
          perm_rows[pos] = t;
          perm_w[pos] = w[(size_t)t * K + j];
          inv_pos[(size_t)t * K + j] = pos;
        }
      }
    }
    __syncthreads();
    if (tid < E) running[tid] += chunk_total[tid];
    __syncthreads();
  }
}

// Many tokens, in two passes over 16-token chunks whose per-expert counts
// the router wrote. Scan: the counts are staged in LDS; wave v prefix-sums
// chunks v, v+16, ... per expert (lane = expert), the 16 wave totals are
// scanned, and each (chunk, expert) gets its first dispatched slot. Wave 0
// then lists the row tiles.
constexpr int kChunk = 16;
constexpr int kScanMaxChunks = 256;  // 4096 tokens per scan pass

__global__ __launch_bounds__(1024) void dispatch_scan_kernel(
    const int* __restrict__ chunk_counts, int nchunks, int T, int E, int K, int bm,
    int* __restrict__ chunk_base, int* __restrict__ offsets, int* __restrict__ tiles,
    int* __restrict__ counters) {
  __shared__ int cc[kScanMaxChunks][64];
  __shared__ int wave_total[16][64];
  __shared__ int expert_total[64];
  __shared__ int carry[64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (tid < 64) carry[tid] = 0;
  // Pass 1: totals per expert over all chunks.
  int mine = 0;
  for (int c = wave; c < nchunks; c += 16) mine += chunk_counts[(size_t)c * 64 + lane];
  wave_total[wave][lane] = mine;
  __syncthreads();
  if (tid < 64) {
    int total = 0;
    for (int v = 0; v < 16; v++) total += wave_total[v][tid];
    expert_total[tid] = tid < E ? total : 0;
  }
  __syncthreads();
  if (wave == 0) {
    const int total = expert_total[lane];
    int incl = total;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    const int excl = incl - total;
    if (lane < E) offsets[lane] = excl;
    if (lane == 0) offsets[E] = T * K;
    carry[lane] = excl;
    const int nt = lane < E ? (total + bm - 1) / bm : 0;
    int tincl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(tincl, o);
      if (lane >= o) tincl += v;
    }
    const int tstart = tincl - nt;
    for (int i = 0; i < nt; i++) {
      tiles[2 * (tstart + i)] = lane;
      tiles[2 * (tstart + i) + 1] = i * bm;
    }
    const int routed_tiles = __shfl(tincl, 63);
    const int shared_tiles = (T + bm - 1) / bm;
    for (int i = lane; i < shared_tiles; i += 64) {
      tiles[2 * (routed_tiles + i)] = E;
      tiles[2 * (routed_tiles + i) + 1] = i * bm;
    }
    if (lane == 0) {
      counters[0] = routed_tiles + shared_tiles;
      counters[1] = routed_tiles;
    }
  }
  __syncthreads();
  // Pass 2: chunk bases, kScanMaxChunks chunks at a time through LDS.
  for (int c0 = 0; c0 < nchunks; c0 += kScanMaxChunks) {
    const int nc = min(kScanMaxChunks, nchunks - c0);
    for (int i = tid; i < nc * 64; i += 1024) cc[i >> 6][i & 63] = chunk_counts[(size_t)c0 * 64 + i];
    __syncthreads();
    // Wave v owns a contiguous run of chunks.
    const int per = (nc + 15) / 16;
    const int cb = wave * per, ce = min(nc, cb + per);
    int run = 0;
    for (int c = cb; c < ce; c++) run += cc[c][lane];
    wave_total[wave][lane] = run;
    __syncthreads();
    int before = carry[lane];
    for (int v = 0; v < wave; v++) before += wave_total[v][lane];
    for (int c = cb; c < ce; c++) {
      chunk_base[(size_t)(c0 + c) * 64 + lane] = before;
      before += cc[c][lane];
    }
    __syncthreads();
    if (tid < 64) {
      int add = 0;
      for (int v = 0; v < 16; v++) add += wave_total[v][tid];
      carry[tid] += add;
    }
    __syncthreads();
  }
}

// Scatter: one wave per chunk (lanes past the chunk idle); a token's rank
// among earlier tokens of the same expert inside the chunk comes from a
// ballot.
__global__ __launch_bounds__(64) void dispatch_scatter_kernel(
    const int* __restrict__ ids, const float* __restrict__ w, int T, int E, int K,
    const int* __restrict__ chunk_base, int* __restrict__ perm_rows, float* __restrict__ perm_w,
    int* __restrict__ inv_pos) {
  const int lane = threadIdx.x;
  const int c = blockIdx.x;
  const int t = c * kChunk + lane;
  const bool valid = lane < kChunk && t < T;
  int my_e[8], my_rank[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    my_e[j] = (valid && j < K) ? ids[(size_t)t * K + j] : -1;
    my_rank[j] = 0;
  }
  const unsigned long long lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int e = 0; e < E; e++) {
    bool has = false;
#pragma unroll
    for (int j = 0; j < 8; j++) has |= my_e[j] == e;
    const unsigned long long mask = __ballot(has);
    if (!mask) continue;
    const int r = __popcll(mask & lt);
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (my_e[j] == e) my_rank[j] = r;
  }
  if (!valid) return;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    if (j < K) {
      const int e = my_e[j];
      const int pos = chunk_base[(size_t)c * 64 + e] + my_rank[j];
      perm_rows[pos] = t;
      perm_w[pos] = w[(size_t)t * K + j];
      inv_pos[(size_t)t * K + j] = pos;
    }
  }
}

void launch_dispatch_chunked(const int* ids, const float* w, int T, int E, int K, int bm,
                             const int* chunk_counts, int* chunk_base, int* offsets,
                             int* perm_rows, float* perm_w, int* inv_pos, int* tiles,
                             int* counters, hipStream_t s) {
  const int nchunks = (T + kChunk - 1) / kChunk;
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), 0, s, chunk_counts, nchunks, T,
                     E, K, bm, chunk_base, offsets, tiles, counters);
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nchunks), dim3(64), 0, s, ids, w, T, E, K,
                     chunk_base, perm_rows, perm_w, inv_pos);
}

void launch_dispatch(const int* ids, const float* w, int T, int E, int K, int bm, int* offsets,
                     int* perm_rows, float* perm_w, int* inv_pos, int* tiles, int* counters,
                     hipStream_t s) {
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispatchThreads), 0, s, ids, w, T, E, K, bm,
                     offsets, perm_rows, perm_w, inv_pos, tiles, counters);
}

}  // namespace uocr
