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

void launch_dispatch(const int* ids, const float* w, int T, int E, int K, int bm, int* offsets,
                     int* perm_rows, float* perm_w, int* inv_pos, int* tiles, int* counters,
                     hipStream_t s) {
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispatchThreads), 0, s, ids, w, T, E, K, bm,
                     offsets, perm_rows, perm_w, inv_pos, tiles, counters);
}

}  // namespace uocr
