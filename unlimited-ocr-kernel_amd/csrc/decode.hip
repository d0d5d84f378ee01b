// One-token (decode) expert engine: bound by the bytes of the active
// experts' weights. Three launches, and no cross-workgroup synchronisation
// inside a launch (kernel boundaries order everything):
//   stage 1  router logits          + shared-expert gate/up  -> h_shared
//   stage 2  routed gate/up         + shared-expert down     -> y_shared
//            (every wave routes the token itself from the E logits)
//   stage 3  routed down of all K experts for an 8-feature block, then the
//            ordered combine of that block.
// Weights are read with range-checked buffer loads (out-of-range chunks
// read as zero without a memory access), all issued before the first use,
// and before the activation row is staged into LDS.
//
// Arithmetic is that of Decoder::projection / feed_forward for one row
// (src/decoder/mod.rs:99-122): BF16 widened exactly; INT8 weight-only as
// the rounded product w * scale (src/cpu/quantized.rs:119-131); W8A8 for
// DynamicActivations (one row is always a single-row group, :103-104) with
// the row quantised per 32-block and exact i32 block sums (:155-236).
// Routing is moe::route (src/decoder/moe.rs:11-31) on logits from
// ops::linear (src/cpu/ops.rs:23-58); the combine follows moe.rs:85-103.
#include "common.hpp"
#include "moe_kernels.hpp"
#include "routing.hpp"
#include "rowdot.hpp"

namespace uocr {

namespace {

constexpr int kWide = 2048;     // widest reduction dimension (H, S)
constexpr int kNarrow = 1024;   // widest routed intermediate size (I)
constexpr int kMaxK = 8;        // most routed experts per token

// Row of w13 holding gate value k (up value k is 32 rows further).
__device__ __forceinline__ int gate_row(int k) { return (k >> 5) * 64 + (k & 31); }

__device__ __forceinline__ int clamp_group(int g, int n) { return g < 0 ? 0 : (g >= n ? n - 1 : g); }

struct RowSmem {
  float xl[kWide];
  int8_t xq[kWide];
  float xs[kWide / kQBlock];
};

template <int KIND>
__device__ __forceinline__ const void* w13_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? (const void*)(L.w13 + L.w13_offset(g))
                       : (const void*)(L.q13 + L.w13_offset(g));
}
template <int KIND>
__device__ __forceinline__ const float* s13_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? nullptr : L.s13 + L.s13_offset(g);
}
template <int KIND>
__device__ __forceinline__ const float* s2_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? nullptr : L.s2 + L.s2_offset(g);
}
template <int KIND>
__device__ __forceinline__ const void* w2_of(const DeviceLayer& L, int g) {
  return KIND == kBF16 ? (const void*)(L.w2 + L.w2_offset(g))
                       : (const void*)(L.q2 + L.w2_offset(g));
}

// Stage 1. Workgroups [0, nr): router rows 8b .. 8b+7 (BF16 router, FP32
// x). Workgroups [nr, nr + S/4): shared-expert hidden values 4b' .. 4b'+3,
// h = silu(gate) * up, into gu[K*I ..].
template <int KIND, int KH>
__global__ __launch_bounds__(64) void decode_stage1_kernel(DeviceLayer L, Scratch S) {
  __shared__ __align__(16) RowSmem sm;
  const int lane = threadIdx.x;
  const int q = lane >> 4;
  const int nr = (L.E + 7) / 8;
  const int b = blockIdx.x;
  if (b < nr) {
    RowPair<kBF16, KH> P;
    const int ra = 8 * b + q, rb = ra + 4;
    issue_rows(P, L.router, nullptr, L.E, L.H, ra, rb);
    RowStage<KH> X;
    load_row(X, S.xn, L.H, lane);
    store_row(X, sm.xl, L.H, lane);
    __syncthreads();
    float r0, r1;
    dot_rows(P, L.H, sm.xl, nullptr, nullptr, r0, r1);
    if ((lane & 15) == 0) {
      if (ra < L.E) S.logits[ra] = r0;
      if (rb < L.E) S.logits[rb] = r1;
    }
    return;
  }
  const int k = 4 * (b - nr) + q;  // shared hidden index (< S by the grid)
  const int ra = gate_row(k);
  RowPair<KIND, KH> P;
  issue_rows(P, w13_of<KIND>(L, L.E), s13_of<KIND>(L, L.E), 2 * L.S, L.H, ra, ra + 32);
  RowStage<KH> X;
  load_row(X, S.xn, L.H, lane);
  store_row(X, sm.xl, L.H, lane);
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    quantize_lds(sm.xl, L.H, sm.xq, sm.xs, lane, S.err);
    __syncthreads();
  }
  float r0, r1;
  dot_rows(P, L.H, sm.xl, sm.xq, sm.xs, r0, r1);
  if ((lane & 15) == 0) S.gu[(size_t)L.K * L.I + k] = silu(r0) * r1;
}

// Stage 2. Workgroups [0, K * I/4): routed hidden values 4b' .. 4b'+3 of
// the expert in ascending slot b / (I/4), into gu[slot * I ..]. Workgroups
// after that: shared-expert down rows 8b' .. 8b'+7 -> ys. Workgroup 0 also
// writes the routing and the one-token dispatch (ids, weights, offsets,
// permutation, row tiles).
template <int KIND, int KH>
__global__ __launch_bounds__(64) void decode_stage2_kernel(DeviceLayer L, Scratch S) {
  __shared__ __align__(16) RowSmem sm;
  __shared__ __align__(16) RouteSmem rs;
  const int lane = threadIdx.x;
  const int q = lane >> 4;
  const int per_expert = L.I / 4;
  const int nrouted = L.K * per_expert;
  const int b = blockIdx.x;
  if (b < nrouted) {
    // The logit load goes first: routing waits for it alone, while the
    // activation row is still in flight.
    const float logit = lane < L.E ? S.logits[lane] : 0.0f;
    RowStage<KH> X;
    load_row(X, S.xn, L.H, lane);
    const LdsRoute r = route_lds(logit, L.E, L.K, rs);
    const int slot = b / per_expert;
    const int g = clamp_group(__builtin_amdgcn_readfirstlane(slot_expert(r.mask, slot)), L.E);
    const int k = 4 * (b - slot * per_expert) + q;
    const int ra = gate_row(k);
    RowPair<KIND, KH> P;
    issue_rows(P, w13_of<KIND>(L, g), s13_of<KIND>(L, g), 2 * L.I, L.H, ra, ra + 32);
    if (b == 0) {
      const float w = route_lds_weight(r, L.K, L.normalize, L.scale, rs);
      if (!r.ok && lane == 0) raise_error(S.err, kErrNumerical);
      const unsigned long long below_mask = r.mask & ((1ull << lane) - 1ull);
      const int asc = __popcll(below_mask);  // ascending slot / selected ids below lane
      if ((r.mask >> lane) & 1ull) {
        S.topk_ids[r.rank] = lane;
        S.topk_w[r.rank] = w;
        S.inv_pos[r.rank] = asc;
        S.perm_rows[asc] = 0;
        S.perm_w[asc] = w;
        S.tiles[2 * asc] = lane;
        S.tiles[2 * asc + 1] = 0;
      }
      if (lane < L.E) S.offsets[lane] = asc;
      if (lane == 0) {
        S.offsets[L.E] = L.K;
        S.tiles[2 * L.K] = L.E;
        S.tiles[2 * L.K + 1] = 0;
        S.counters[0] = L.K + 1;
        S.counters[1] = L.K;
      }
    }
    store_row(X, sm.xl, L.H, lane);
    __syncthreads();
    if constexpr (KIND == kW8A8) {
      quantize_lds(sm.xl, L.H, sm.xq, sm.xs, lane, S.err);
      __syncthreads();
    }
    float r0, r1;
    dot_rows(P, L.H, sm.xl, sm.xq, sm.xs, r0, r1);
    if ((lane & 15) == 0) S.gu[(size_t)slot * L.I + k] = silu(r0) * r1;
    return;
  }
  const int ra = 8 * (b - nrouted) + q, rb = ra + 4;
  RowPair<KIND, kWide> P;
  issue_rows(P, w2_of<KIND>(L, L.E), s2_of<KIND>(L, L.E), L.H, L.S, ra, rb);
  RowStage<kWide> Hs;
  load_row(Hs, S.gu + (size_t)L.K * L.I, L.S, lane);
  store_row(Hs, sm.xl, L.S, lane);
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    quantize_lds(sm.xl, L.S, sm.xq, sm.xs, lane, S.err);
    __syncthreads();
  }
  float r0, r1;
  dot_rows(P, L.S, sm.xl, sm.xq, sm.xs, r0, r1);
  if ((lane & 15) == 0) {
    if (ra < L.H) S.ys[ra] = r0;
    if (rb < L.H) S.ys[rb] = r1;
  }
}

struct Stage3Smem {
  float hl[kMaxK][kNarrow];
  int8_t hq[kMaxK][kNarrow];
  float hs[kMaxK][kNarrow / kQBlock];
  float yl[kMaxK][8];
};

// Stage 3: one workgroup per 8 output features, wave w = routed expert in
// ascending slot w, then the ordered combine of the 8 features:
// out = (residual +) (ys + p_0 y_0 + p_1 y_1 + ...), mul then add.
template <int KIND>
__global__ __launch_bounds__(64 * kMaxK) void decode_stage3_kernel(DeviceLayer L, Scratch S,
                                                                   const float* residual,
                                                                   float* out) {
  __shared__ __align__(16) Stage3Smem sm;
  // Wave-uniform (scalar) so the per-wave buffer bases stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int f0 = 8 * blockIdx.x;
  // Hidden row first, then the expert id (scalar load) and its weights;
  // the combine inputs are loaded now and used last.
  RowStage<kNarrow> Hr;
  load_row(Hr, S.gu + (size_t)wave * L.I, L.I, lane);
  const int g = clamp_group(__builtin_amdgcn_readfirstlane(S.tiles[2 * wave]), L.E);
  const int ra = f0 + q, rb = ra + 4;
  RowPair<KIND, kNarrow> P;
  issue_rows(P, w2_of<KIND>(L, g), s2_of<KIND>(L, g), L.H, L.I, ra, rb);
  const float ys_f = S.ys[f0 + (lane & 7)];
  const float res_f = residual ? residual[f0 + (lane & 7)] : 0.0f;
  float pw[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK; j++) pw[j] = j < L.K ? S.perm_w[j] : 0.0f;
  store_row(Hr, sm.hl[wave], L.I, lane);
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    quantize_lds(sm.hl[wave], L.I, sm.hq[wave], sm.hs[wave], lane, S.err);
    __syncthreads();
  }
  float r0, r1;
  dot_rows(P, L.I, sm.hl[wave], sm.hq[wave], sm.hs[wave], r0, r1);
  if ((lane & 15) == 0) {
    sm.yl[wave][q] = r0;
    sm.yl[wave][q + 4] = r1;
  }
  __syncthreads();
  if (wave == 0 && lane < 8) {
    float acc = ys_f;
#pragma unroll
    for (int j = 0; j < kMaxK; j++)
      if (j < L.K) acc = acc + pw[j] * sm.yl[j][lane];
    if (residual) acc = res_f + acc;
    out[f0 + lane] = acc;
  }
}

template <int KIND, int KH>
void launch_stage(int stage, const DeviceLayer& L, const Scratch& S, const float* residual,
                  float* out, hipStream_t s) {
  if (stage == 1)
    decode_stage1_kernel<KIND, KH><<<dim3((L.E + 7) / 8 + L.S / 4), dim3(64), 0, s>>>(L, S);
  else if (stage == 2)
    decode_stage2_kernel<KIND, KH><<<dim3(L.K * (L.I / 4) + L.H / 8), dim3(64), 0, s>>>(L, S);
  else
    decode_stage3_kernel<KIND><<<dim3(L.H / 8), dim3(64 * L.K), 0, s>>>(L, S, residual, out);
}

template <int KH>
void launch_kind(int stage, const DeviceLayer& L, const Scratch& S, const float* residual,
                 float* out, hipStream_t s) {
  if (L.quant_mode == 0)
    launch_stage<kBF16, KH>(stage, L, S, residual, out, s);
  else if (L.quant_mode == 1)
    launch_stage<kInt8, KH>(stage, L, S, residual, out, s);
  else
    launch_stage<kW8A8, KH>(stage, L, S, residual, out, s);
}

}  // namespace

bool decode_supported(const DeviceLayer& L) {
  // Stage 1/2 rows reduce over H (<= 2048) and S (<= 2048); stage 3 over
  // I (<= 1024) with one wave per routed expert; routing is one wave.
  return L.H <= kWide && L.S <= kWide && L.I <= kNarrow && L.K >= 1 && L.K <= kMaxK &&
         L.E <= 64 && L.H % 8 == 0 && L.I % 4 == 0 && L.S % 4 == 0;
}

void launch_decode_stage(int stage, const DeviceLayer& L, const Scratch& S, const float* residual,
                         float* out, hipStream_t s) {
  if (L.H <= 1280)
    launch_kind<1280>(stage, L, S, residual, out, s);
  else
    launch_kind<kWide>(stage, L, S, residual, out, s);
}

}  // namespace uocr
