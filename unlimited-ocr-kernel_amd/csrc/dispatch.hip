// Dispatch: per-expert histogram, exclusive prefix sum and a stable
// permutation of (token, slot) assignments into expert-major order, tokens
// ascending within an expert.
//
// Reference: Decoder::experts pushes (row, p) onto assignments[expert] while
// walking rows in order (src/decoder/mod.rs:127-141) and then visits experts
// in ascending id (:198-218); the permutation below is that order.
#include "common.hpp"
#include "moe_kernels.hpp"
#include "rowdot.hpp"

namespace uocr {

int max_tiles(int T, int K, int E, int bm) {
  // Routed: sum_e ceil(n_e / bm) <= min(E, T*K) + T*K / bm. Shared: ceil(T / bm).
  long long tk = (long long)T * K;
  long long routed = (tk < E ? tk : E) + tk / bm;
  return (int)(routed + (T + bm - 1) / bm);
}

constexpr int kDispatchThreads = 1024;
constexpr int kDispatchWaves = kDispatchThreads / 64;

// Row tiles, written by one wave: lane e holds expert e's row count c (0
// past E). Routed tiles of bm rows go expert-major into a first list; when
// narrow > 0, an expert's last tile of at most `narrow` rows goes instead to
// a second list placed after the first (the MFMA engine runs those as
// 128 x 512 items); the shared expert's tiles follow. counters: [0] all
// tiles, [1] routed tiles, [2] end of the first list.
__device__ void write_tiles(int lane, int c, int T, int bm, int narrow,
                            int* __restrict__ tiles, int* __restrict__ counters, int shared_group) {
  const int full = c / bm, rem = c - full * bm;
  const bool nar = narrow > 0 && rem > 0 && rem <= narrow;
  const int nsq = full + ((rem > 0 && !nar) ? 1 : 0);
  // Two counts in one scan: square tiles < 2^16, narrow ones <= 64.
  const int packed = nsq | ((nar ? 1 : 0) << 16);
  int incl = packed;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  const int excl = incl - packed;
  const int total = __shfl(incl, 63);
  const int routed_sq = total & 0xffff, routed_nr = total >> 16;
  const int routed_tiles = routed_sq + routed_nr;
  const int sq0 = excl & 0xffff, nr0 = excl >> 16;
  for (int i = 0; i < nsq; i++) {
    tiles[2 * (sq0 + i)] = lane;
    tiles[2 * (sq0 + i) + 1] = i * bm;
  }
  if (nar) {
    tiles[2 * (routed_sq + nr0)] = lane;
    tiles[2 * (routed_sq + nr0) + 1] = full * bm;
  }
  const int shared_tiles = (T + bm - 1) / bm;
  for (int i = lane; i < shared_tiles; i += 64) {
    tiles[2 * (routed_tiles + i)] = shared_group;
    tiles[2 * (routed_tiles + i) + 1] = i * bm;
  }
  if (lane == 0) {
    counters[0] = routed_tiles + shared_tiles;
    counters[1] = routed_tiles;
    counters[2] = routed_sq;
  }
}

// One workgroup. Tokens are taken 1024 at a time (one per thread); inside a
// wave the rank of a token among earlier tokens of the same expert comes
// from a ballot, across waves from an LDS prefix, across chunks from a
// running count — together the stable counting sort.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(
    const int* __restrict__ ids, const float* __restrict__ w, int T, int E, int K, int bm,
    int narrow, int* __restrict__ offsets, int* __restrict__ perm_rows, float* __restrict__ perm_w,
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
    write_tiles(lane, c, T, bm, narrow, tiles, counters, E);
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
constexpr int kChunk = 16;          // tokens per router chunk
constexpr int kFusedThreads = 256;  // 16 chunk rows x 16 expert quads per pass

// Dispatch for the chunked router (one workgroup per 16-token chunk, no
// second launch): every workgroup sums the router's per-chunk expert counts
// over all chunks (the expert totals, hence the expert offsets) and over
// the chunks before its own (its chunk's first slot per expert), then
// places its tokens: a token's rank among earlier tokens of the same expert
// inside the chunk comes from a per-expert token mask. Workgroup 0 also writes the offsets,
// the row tiles and the tile counters. The slot of (token t, expert e) is
// offsets[e] + (count of e in earlier chunks) + (rank of t in its chunk):
// tokens in ascending order within each expert, as the reference's stable
// dispatch (src/decoder/mod.rs:124-183).
__global__ __launch_bounds__(kFusedThreads) void dispatch_fused_kernel(
    const int* __restrict__ chunk_counts, const int* __restrict__ ids, const float* __restrict__ w,
    int nchunks, int T, int E, int K, int bm, int narrow, int* __restrict__ offsets,
    int* __restrict__ perm_rows, float* __restrict__ perm_w, int* __restrict__ inv_pos,
    int* __restrict__ tiles, int* __restrict__ counters) {
  __shared__ __attribute__((aligned(16))) int part_tot[16][64];
  __shared__ __attribute__((aligned(16))) int part_bef[16][64];
  __shared__ int base[64];
  __shared__ unsigned long long emask[64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Raised issue priority, as the router's: this launch shares CUs with the
  // shared expert's GEMM on a two-stream forward.
  __builtin_amdgcn_s_setprio(3);
  const int c = blockIdx.x;
  // Wave 0's lanes < 16 own the chunk's tokens; their selections and
  // weights are loaded first, in flight while the counts are summed.
  const int t = c * kChunk + lane;
  const bool valid = wave == 0 && lane < kChunk && t < T;
  int my_e[8];
  float my_w[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    my_e[j] = (valid && j < K) ? ids[(size_t)t * K + j] : -1;
    my_w[j] = (valid && j < K) ? w[(size_t)t * K + j] : 0.0f;
  }
  // Thread (row = tid / 16, quad = tid % 16) sums experts 4 quad .. 4 quad + 3
  // of chunks row, row + 16, ...; 16 loads in flight per pass, chunks past
  // the end read as zero.
  const int row = tid >> 4, quad = tid & 15;
  const __amdgpu_buffer_rsrc_t cr = make_rsrc(chunk_counts, (uint32_t)nchunks * 64u * 4u);
  u32x4 tot = {0u, 0u, 0u, 0u}, bef = {0u, 0u, 0u, 0u};
  for (int c0 = 0; c0 < nchunks; c0 += 256) {
    u32x4 v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t cc = (uint32_t)(c0 + 16 * i + row);
      v[i] = __builtin_amdgcn_raw_buffer_load_b128(cr, (cc * 64u + 4u * quad) * 4u, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
      tot += v[i];
      if (c0 + 16 * i + row < c) bef += v[i];
    }
  }
  *reinterpret_cast<u32x4*>(&part_tot[row][4 * quad]) = tot;
  *reinterpret_cast<u32x4*>(&part_bef[row][4 * quad]) = bef;
  __syncthreads();
  if (wave == 0) {
    int total = 0, before = 0;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      total += part_tot[r][lane];
      before += part_bef[r][lane];
    }
    if (lane >= E) total = 0;
    int incl = total;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    const int excl = incl - total;
    base[lane] = excl + before;
    if (c == 0) {
      if (lane < E) offsets[lane] = excl;
      if (lane == 0) offsets[E] = T * K;
      write_tiles(lane, total, T, bm, narrow, tiles, counters, E);
    }
  }
  if (tid < 64) emask[tid] = 0ull;
  __syncthreads();
  if (wave != 0) return;
  // Place the chunk's tokens (lanes past the chunk idle): bit t of emask[e]
  // is set when token t of the chunk selected expert e, so a token's rank
  // among the chunk's earlier tokens of that expert is a popcount. One wave
  // sets and reads the masks: a wavefront-scope release/acquire pair around
  // a wave barrier orders every lane's atomicOr before any lane's read.
#pragma unroll
  for (int j = 0; j < 8; j++)
    if (my_e[j] >= 0) atomicOr(&emask[my_e[j]], 1ull << lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (!valid) return;
  const unsigned long long lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int j = 0; j < 8; j++) {
    if (j < K) {
      const int e = my_e[j];
      const int pos = base[e] + __popcll(emask[e] & lt);
      perm_rows[pos] = t;
      perm_w[pos] = my_w[j];
      inv_pos[(size_t)t * K + j] = pos;
    }
  }
}

void launch_dispatch_chunked(const int* ids, const float* w, int T, int E, int K, int bm,
                             int narrow, const int* chunk_counts, int* offsets, int* perm_rows, float* perm_w,
                             int* inv_pos, int* tiles, int* counters, hipStream_t s) {
  const int nchunks = (T + kChunk - 1) / kChunk;
  hipLaunchKernelGGL(dispatch_fused_kernel, dim3(nchunks), dim3(kFusedThreads), 0, s, chunk_counts,
                     ids, w, nchunks, T, E, K, bm, narrow, offsets, perm_rows, perm_w, inv_pos,
                     tiles, counters);
}

void launch_dispatch(const int* ids, const float* w, int T, int E, int K, int bm, int narrow,
                     int* offsets,
                     int* perm_rows, float* perm_w, int* inv_pos, int* tiles, int* counters,
                     hipStream_t s) {
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispatchThreads), 0, s, ids, w, T, E, K, bm,
                     narrow, offsets, perm_rows, perm_w, inv_pos, tiles, counters);
}

}  // namespace uocr
