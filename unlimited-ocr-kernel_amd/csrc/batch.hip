// Small-batch expert engine: row tiles of up to 16 tokens of one expert
// group (the shared expert is group E). Every workgroup streams a slice of
// the group's weight rows once, with all of its loads in flight, and dots it
// with the tile's activation rows staged in LDS. Used for 2 <= T <= 16 and
// for INT8 weights at any T (tiles of 16 rows).
//
// Also the fence-free small-batch router (2 <= T <= 16): logits, then one
// workgroup that routes every token and builds the dispatch.
//
// Arithmetic: Decoder::projection / feed_forward (src/decoder/mod.rs:
// 99-122) per row; INT8 weight-only as the rounded w * scale in FP32; W8A8
// only for DynamicActivations groups of a single row (:103-104).
#include "common.hpp"
#include "moe_kernels.hpp"
#include "routing.hpp"
#include "rowdot.hpp"

namespace uocr {

namespace {

constexpr int kTileRows = kGemvChunk;  // tokens per row tile
constexpr int kDotTok = 8;             // tokens per register batch of the dot
constexpr int kStage = 15360;        // FP32 activations staged per workgroup (60 KiB)
constexpr int kWideK = 2048;         // widest reduction dimension (H, S)
constexpr int kNarrowK = 1024;       // widest routed expert width (I)

struct TileInfo {
  int g, r0, n, group_rows;
  bool routed;
};

// singles: only routed groups of a single row (the W8A8 rows the MFMA engine
// leaves to this engine under DynamicActivations).
__device__ __forceinline__ bool load_tile(const DeviceLayer& L, const Scratch& S, int T,
                                          int mchunk, int singles, TileInfo& ti) {
  const int tile = blockIdx.y;
  if (tile >= S.counters[0]) return false;
  ti.g = S.tiles[2 * tile];
  ti.r0 = S.tiles[2 * tile + 1];
  ti.routed = ti.g < L.E;
  ti.group_rows = ti.routed ? S.offsets[ti.g + 1] - S.offsets[ti.g] : T;
  if (singles && !(ti.routed && ti.group_rows == 1)) return false;
  ti.n = min(mchunk, ti.group_rows - ti.r0);
  return ti.n > 0;
}

// Row of w13 holding gate value k (up value k is 32 rows further).
__device__ __forceinline__ int gate_row(int k) { return (k >> 5) * 64 + (k & 31); }

struct BatchSmem {
  float x[kStage];
  int8_t xq[kWideK];
  float xs[kWideK / kQBlock];
  const float* rows[kTileRows];
};

// Stages activation rows [b0, b0 + nb) of the tile into LDS (row-major,
// stride K) with every thread; `row_of(t)` gives the source row pointer.
template <typename RowOf>
__device__ __forceinline__ void stage_tile(BatchSmem& sm, int b0, int nb, int K, RowOf row_of) {
  if (threadIdx.x < nb) sm.rows[threadIdx.x] = row_of(b0 + threadIdx.x);
  __syncthreads();
  const int vec = K / 4;
  const int total = nb * vec;
  constexpr int kPer = 8;
  for (int base = 0; base < total; base += kPer * 256) {
    u32x4 v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int at = base + threadIdx.x + i * 256;
      if (at < total) {
        const int t = at / vec;
        v[i] = reinterpret_cast<const u32x4*>(sm.rows[t])[at - t * vec];
      }
    }
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int at = base + threadIdx.x + i * 256;
      if (at < total) reinterpret_cast<u32x4*>(sm.x)[at] = v[i];
    }
  }
  __syncthreads();
}

template <int KIND>
__device__ __forceinline__ const void* w13_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? (const void*)(L.w13 + L.w13_offset(g))
                       : (const void*)(L.q13 + L.w13_offset(g));
}
template <int KIND>
__device__ __forceinline__ const void* w2_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? (const void*)(L.w2 + L.w2_offset(g))
                       : (const void*)(L.q2 + L.w2_offset(g));
}
template <int KIND>
__device__ __forceinline__ const float* s13_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? nullptr : L.s13 + L.s13_offset(g);
}
template <int KIND>
__device__ __forceinline__ const float* s2_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? nullptr : L.s2 + L.s2_offset(g);
}

// Dots the loaded rows with the tile's activations in token batches that fit
// the LDS budget; emit(t, r0, r1) receives every token's two row sums (in
// every lane of the row's 16-lane group). A single-row tile of an INT8
// layer in DynamicActivations mode takes the W8A8 dot instead.
template <int KIND, int KMAX, typename RowOf, typename Emit>
__device__ __forceinline__ void tile_dot(const DeviceLayer& L, const Scratch& S, BatchSmem& sm,
                                         const RowPair<KIND, KMAX>& P, int K, const TileInfo& ti,
                                         RowOf row_of, Emit emit) {
  const int lane = threadIdx.x & 63;
  if constexpr (KIND == kInt8) {
    if (L.quant_mode == 2 && ti.group_rows == 1) {
      stage_tile(sm, 0, 1, K, row_of);
      if (threadIdx.x < 64) quantize_lds(sm.x, K, sm.xq, sm.xs, lane, S.err);
      __syncthreads();
      float r0, r1;
      dot_rows_as<kW8A8>(P, K, sm.x, sm.xq, sm.xs, r0, r1);
      emit(0, r0, r1);
      return;
    }
  }
  // Tokens staged per pass (LDS budget), dotted kDotTok at a time; the
  // weight rows stay in registers throughout.
  const int per = kStage / K < kTileRows ? kStage / K : kTileRows;
  for (int b0 = 0; b0 < ti.n; b0 += per) {
    const int nb = min(per, ti.n - b0);
    if (b0 > 0) __syncthreads();  // the previous pass is consumed
    stage_tile(sm, b0, nb, K, row_of);
    for (int d0 = 0; d0 < nb; d0 += kDotTok) {
      const int nd = min(kDotTok, nb - d0);
      float a0[kDotTok], a1[kDotTok];
#pragma unroll
      for (int t = 0; t < kDotTok; t++) a0[t] = a1[t] = 0.0f;
      dot_rows_multi(P, K, sm.x + d0 * K, K, nd, a0, a1);
#pragma unroll
      for (int t = 0; t < kDotTok; t++)
        if (t < nd) emit(b0 + d0 + t, row16_sum(a0[t]), row16_sum(a1[t]));
    }
  }
}

// Gate/up: blockIdx.y = row tile, blockIdx.x = 16 hidden values (each wave
// 4 gate rows and the 4 matching up rows). h = silu(gate) * up
// (Decoder::feed_forward, src/decoder/mod.rs:114-122).
template <int KIND, int KH>
__global__ __launch_bounds__(256) void batch_gateup_kernel(DeviceLayer L, Scratch S, int T,
                                                           int mchunk, int singles) {
  __shared__ __align__(16) BatchSmem sm;
  TileInfo ti;
  if (!load_tile(L, S, T, mchunk, singles, ti)) return;
  const int W = L.width(ti.g);
  const int k0 = 16 * blockIdx.x;
  if (k0 >= W) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = k0 + 4 * wave + (lane >> 4);
  const int ra = gate_row(k);
  RowPair<KIND, KH> P;
  issue_rows(P, w13_of<KIND>(L, ti.g), s13_of<KIND>(L, ti.g), 2 * W, L.H, ra, ra + 32);
  const int base = ti.routed ? S.offsets[ti.g] + ti.r0 : ti.r0;
  auto row_of = [&](int t) {
    const int row = ti.routed ? S.perm_rows[base + t] : base + t;
    return S.xn + (size_t)row * L.H;
  };
  float* hout = ti.routed ? S.h + (size_t)base * L.I : S.hs + (size_t)base * L.S;
  const int ld = ti.routed ? L.I : L.S;
  tile_dot(L, S, sm, P, L.H, ti, row_of, [&](int t, float g, float u) {
    if ((lane & 15) == 0) hout[(size_t)t * ld + k] = silu(g) * u;
  });
}

// Down: blockIdx.y = row tile, blockIdx.x = 32 output features (each wave
// 8 rows of the down matrix). Writes y (routed, dispatched order) or ys.
template <int KIND, int KMAX>
__device__ __forceinline__ void down_body(const DeviceLayer& L, const Scratch& S, BatchSmem& sm,
                                          const TileInfo& ti) {
  const int W = L.width(ti.g);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ra = 32 * blockIdx.x + 8 * wave + (lane >> 4), rb = ra + 4;
  RowPair<KIND, KMAX> P;
  issue_rows(P, w2_of<KIND>(L, ti.g), s2_of<KIND>(L, ti.g), L.H, W, ra, rb);
  const int base = ti.routed ? S.offsets[ti.g] + ti.r0 : ti.r0;
  const float* hin = ti.routed ? S.h + (size_t)base * L.I : S.hs + (size_t)base * L.S;
  auto row_of = [&](int t) { return hin + (size_t)t * W; };
  float* yout = ti.routed ? S.y + (size_t)base * L.H : S.ys + (size_t)base * L.H;
  tile_dot(L, S, sm, P, W, ti, row_of, [&](int t, float y0, float y1) {
    if ((lane & 15) == 0) {
      if (ra < L.H) yout[(size_t)t * L.H + ra] = y0;
      if (rb < L.H) yout[(size_t)t * L.H + rb] = y1;
    }
  });
}

template <int KIND>
__global__ __launch_bounds__(256) void batch_down_kernel(DeviceLayer L, Scratch S, int T,
                                                         int mchunk, int singles) {
  __shared__ __align__(16) BatchSmem sm;
  TileInfo ti;
  if (!load_tile(L, S, T, mchunk, singles, ti)) return;
  if (ti.routed && L.I <= kNarrowK)
    down_body<KIND, kNarrowK>(L, S, sm, ti);
  else
    down_body<KIND, kWideK>(L, S, sm, ti);
}

// ------------------------------------------------------------- small router

// Logits for T <= 16 tokens: one wave per (8 router rows, 2 tokens), so
// the 2·H·E·T flops spread over E/8 · T/2 workgroups; the router rows are
// read from L2 by every token pair.
constexpr int kRouterTok = 2;

template <int KH>
__global__ __launch_bounds__(64) void small_router_kernel(const float* __restrict__ x,
                                                          DeviceLayer L, Scratch S, int T) {
  __shared__ __align__(16) float xl[kRouterTok * KH];
  const int lane = threadIdx.x;
  const int ra = 8 * blockIdx.x + (lane >> 4), rb = ra + 4;
  const int t0 = kRouterTok * blockIdx.y;
  const int nt = min(kRouterTok, T - t0);
  RowPair<kBF16, KH> P;
  issue_rows(P, L.router, nullptr, L.E, L.H, ra, rb);
  RowStage<kRouterTok * KH> X;
  load_row(X, x + (size_t)t0 * L.H, nt * L.H, lane);
  store_row(X, xl, nt * L.H, lane);
  __syncthreads();
  float a0[kRouterTok], a1[kRouterTok];
#pragma unroll
  for (int t = 0; t < kRouterTok; t++) a0[t] = a1[t] = 0.0f;
  dot_rows_multi(P, L.H, xl, L.H, nt, a0, a1);
#pragma unroll
  for (int t = 0; t < kRouterTok; t++) {
    if (t < nt) {
      const float v0 = row16_sum(a0[t]), v1 = row16_sum(a1[t]);
      if ((lane & 15) == 0) {
        if (ra < L.E) S.logits[(size_t)(t0 + t) * L.E + ra] = v0;
        if (rb < L.E) S.logits[(size_t)(t0 + t) * L.E + rb] = v1;
      }
    }
  }
}

// One workgroup of 16 waves: wave t routes token t (moe::route,
// src/decoder/moe.rs:11-31), then the dispatch of Decoder::experts
// (src/decoder/mod.rs:127-141): per expert, its tokens in ascending order;
// one row tile per active expert and one for the shared expert.
constexpr int kRouteWaves = 16;

__global__ __launch_bounds__(64 * kRouteWaves) void small_route_dispatch_kernel(DeviceLayer L,
                                                                               Scratch S, int T) {
  __shared__ RouteSmem rs[kRouteWaves];
  __shared__ unsigned long long masks[kRouteWaves];
  __shared__ int count[64];
  __shared__ int start[65];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = L.E, K = L.K;
  const bool mine = wave < T;
  // Waves past T route a neutral row (their result is not used).
  const float v = mine && lane < E ? S.logits[(size_t)wave * E + lane] : 0.0f;
  const LdsRoute r = route_wave_lds(v, E, K, rs[wave]);
  const float w = route_wave_weight(r, K, L.normalize, L.scale, rs[wave]);
  if (mine && !r.ok && lane == 0) raise_error(S.err, kErrNumerical);
  if (lane == 0) masks[wave] = mine ? r.mask : 0ull;
  __syncthreads();
  if (wave == 0) {
    int c = 0;
    for (int t = 0; t < T; t++) c += (int)((masks[t] >> lane) & 1ull);
    count[lane] = lane < E ? c : 0;
    int incl = count[lane];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o);
      if (lane >= o) incl += u;
    }
    start[lane] = incl - count[lane];
    if (lane == 63) start[64] = incl;
  }
  __syncthreads();
  if (mine && ((r.mask >> lane) & 1ull)) {
    // Position of (token `wave`, expert `lane`): the expert's start plus the
    // earlier tokens that chose it.
    int before = 0;
    for (int t = 0; t < wave; t++) before += (int)((masks[t] >> lane) & 1ull);
    const int pos = start[lane] + before;
    S.topk_ids[(size_t)wave * K + r.rank] = lane;
    S.topk_w[(size_t)wave * K + r.rank] = w;
    S.inv_pos[(size_t)wave * K + r.rank] = pos;
    S.perm_rows[pos] = wave;
    S.perm_w[pos] = w;
  }
  if (wave == 0) {
    if (lane < E) S.offsets[lane] = start[lane];
    if (lane == 0) S.offsets[E] = T * K;
    // One tile per active expert (<= 16 rows each), ascending id, then the
    // shared expert's.
    const bool active = lane < E && count[lane] > 0;
    const unsigned long long am = __ballot(active);
    const int slot = __popcll(am & ((1ull << lane) - 1ull));
    if (active) {
      S.tiles[2 * slot] = lane;
      S.tiles[2 * slot + 1] = 0;
    }
    const int n_active = __popcll(am);
    if (lane == 0) {
      S.tiles[2 * n_active] = E;
      S.tiles[2 * n_active + 1] = 0;
      S.counters[0] = n_active + 1;
      S.counters[1] = n_active;
    }
  }
}

template <int KIND>
void launch_gateup_kind(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound,
                        int mchunk, int singles, hipStream_t s) {
  const dim3 grid(((singles ? L.I : L.S) + 15) / 16, tiles_bound);
  if (L.H <= 1280)
    batch_gateup_kernel<KIND, 1280><<<grid, dim3(256), 0, s>>>(L, S, T, mchunk, singles);
  else
    batch_gateup_kernel<KIND, kWideK><<<grid, dim3(256), 0, s>>>(L, S, T, mchunk, singles);
}

}  // namespace

bool batch_supported(const DeviceLayer& L) {
  return L.H <= kWideK && L.S <= kWideK && L.I % 16 == 0 && L.H % 32 == 0;
}

void launch_batch_gateup(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound,
                         int mchunk, hipStream_t s, bool singles) {
  if (L.quant_mode == 0)
    launch_gateup_kind<kBF16>(L, S, T, tiles_bound, mchunk, singles, s);
  else
    launch_gateup_kind<kInt8>(L, S, T, tiles_bound, mchunk, singles, s);
}

void launch_batch_down(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound, int mchunk,
                       hipStream_t s, bool singles) {
  const dim3 grid(L.H / 32, tiles_bound);
  if (L.quant_mode == 0)
    batch_down_kernel<kBF16><<<grid, dim3(256), 0, s>>>(L, S, T, mchunk, singles);
  else
    batch_down_kernel<kInt8><<<grid, dim3(256), 0, s>>>(L, S, T, mchunk, singles);
}

void launch_small_route(const float* x, const DeviceLayer& L, const Scratch& S, int T,
                        hipStream_t s) {
  const dim3 grid((L.E + 7) / 8, (T + kRouterTok - 1) / kRouterTok);
  if (L.H <= 1280)
    small_router_kernel<1280><<<grid, dim3(64), 0, s>>>(x, L, S, T);
  else
    small_router_kernel<kWideK><<<grid, dim3(64), 0, s>>>(x, L, S, T);
  small_route_dispatch_kernel<<<dim3(1), dim3(64 * kRouteWaves), 0, s>>>(L, S, T);
}

}  // namespace uocr
