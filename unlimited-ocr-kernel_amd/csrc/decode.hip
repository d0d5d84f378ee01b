// One-token (decode) expert engine: bound by the bytes of the active
// experts' weights. Two launches, and no cross-workgroup synchronisation
// inside a launch (the kernel boundary orders them):
//   gate/up  shared-expert workgroups stream their gate/up rows at once;
//            routed workgroups first compute all E router logits
//            themselves (the router is 160 KiB, read from L2 by every
//            routed workgroup, instead of a launch of its own and a
//            dependent read of its output), route the token in LDS, and
//            stream the gate/up rows of the expert of their slot
//   down     routed down of all K experts and the shared-expert down for an
//            8-feature block, then the ordered combine of that block.
// Weights are read with range-checked buffer loads (out-of-range chunks
// read as zero without a memory access), all issued before the first use,
// and before the activation row is staged into LDS.
//
// Arithmetic is that of Decoder::projection / feed_forward for one row
// (src/decoder/mod.rs:99-122): BF16 widened exactly; INT8 weight-only as
// the rounded product w * scale (src/cpu/quantized.rs:119-131); W8A8 for
// DynamicActivations (one row is always a single-row group, :103-104) with
// the row quantised per 32-block and exact i32 block sums (:155-236).
// Routing is moe::route (src/decoder/moe.rs:7-30) on logits from
// ops::linear (src/cpu/ops.rs:9-59); the combine follows src/decoder/mod.rs:185-194.
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

constexpr int kUpWaves = 8;                     // waves per gate/up workgroup
constexpr int kHidPerWg = kUpWaves * 4;         // hidden values per gate/up workgroup

struct GateUpSmem {
  float xl[kWide];
  int8_t xq[kWide];
  float xs[kWide / kQBlock];
  float logits[64];
  unsigned long long mask;
};

// Stages the activation row (wave 0) into LDS, quantised per 32-block for
// W8A8; the caller's loads stay in flight meanwhile.
template <int KIND, int KH>
__device__ __forceinline__ void stage_x(const DeviceLayer& L, const Scratch& S, GateUpSmem& sm,
                                        int wave, int lane) {
  if (wave == 0) {
    RowStage<KH> X;
    load_row(X, S.xn, L.H, lane);
    store_row(X, sm.xl, L.H, lane);
  }
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    if (wave == 0) quantize_lds(sm.xl, L.H, sm.xq, sm.xs, lane, S.err);
    __syncthreads();
  }
}

// Gate/up. Workgroups [0, S/32): shared-expert hidden values 32b .. 32b+31
// (4 per wave: its 4 gate rows and the 4 matching up rows), h =
// silu(gate) * up into gu[K*I ..]. Workgroups after that: routed slot
// s = b' / (I/32), hidden values 32 (b' % (I/32)) .., into gu[s * I ..];
// the first routed workgroup also writes the logits, the routing and the
// one-token dispatch (ids, weights, offsets, permutation, row tiles).
template <int KIND, int KH>
__global__ __launch_bounds__(64 * kUpWaves) void decode_gateup_kernel(DeviceLayer L, Scratch S) {
  __shared__ __align__(16) GateUpSmem sm;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int n_shared = L.S / kHidPerWg;
  const int per_expert = L.I / kHidPerWg;
  const int b = blockIdx.x;
  if (b < n_shared) {
    const int k = b * kHidPerWg + 4 * wave + q;
    const int ra = gate_row(k);
    RowPair<KIND, KH> P;
    issue_rows(P, w13_of<KIND>(L, L.E), s13_of<KIND>(L, L.E), 2 * L.S, L.H, ra, ra + 32);
    stage_x<KIND, KH>(L, S, sm, wave, lane);
    BlockSumOut bs;
    if (KIND == kW8A8 && S.q8.s_gateup) {
      const int nb = L.H / kQBlock;
      bs.a = S.q8.s_gateup + (size_t)k * nb;
      bs.b = S.q8.s_gateup + (size_t)(L.S + k) * nb;
      bs.na = bs.nb = nb;
    }
    float r0, r1;
    dot_rows(P, L.H, sm.xl, sm.xq, sm.xs, r0, r1, bs);
    if ((lane & 15) == 0) S.gu[(size_t)L.K * L.I + k] = silu(r0) * r1;
    return;
  }
  const int rb = b - n_shared;
  const int slot = rb / per_expert;
  // Router rows 8 wave + q and 8 wave + q + 4 (BF16 router, FP32 x; rows
  // past E read as zero), then the logits into LDS.
  {
    RowPair<kBF16, KH> R;
    issue_rows(R, L.router, nullptr, L.E, L.H, 8 * wave + q, 8 * wave + q + 4);
    stage_x<KIND, KH>(L, S, sm, wave, lane);
    float r0, r1;
    dot_rows(R, L.H, sm.xl, nullptr, nullptr, r0, r1);
    if ((lane & 15) == 0) {
      sm.logits[8 * wave + q] = r0;
      sm.logits[8 * wave + q + 4] = r1;
    }
  }
  __syncthreads();
  // Wave 0 routes the token and publishes the selection; the first routed
  // workgroup's wave 0 also writes the logits, the routing and the
  // one-token dispatch (ids, weights, offsets, permutation, row tiles).
  if (wave == 0) {
    const WaveSel r = route_wave_sel(sm.logits[lane], L.E, L.K);
    if (lane == 0) sm.mask = r.mask;
    if (rb == 0) {
      const float w = route_weight(r, L.normalize, L.scale);
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
      if (lane < L.E) {
        S.offsets[lane] = asc;
        S.logits[lane] = sm.logits[lane];
      }
      if (lane == 0) {
        S.offsets[L.E] = L.K;
        S.tiles[2 * L.K] = L.E;
        S.tiles[2 * L.K + 1] = 0;
        S.counters[0] = L.K + 1;
        S.counters[1] = L.K;
        S.counters[2] = L.K;
        S.counters[3] = L.K;
      }
    }
  }
  __syncthreads();
  const int g = clamp_group(__builtin_amdgcn_readfirstlane(slot_expert(sm.mask, slot)), L.E);
  const int k = kHidPerWg * (rb - slot * per_expert) + 4 * wave + q;
  const int ra = gate_row(k);
  RowPair<KIND, KH> P;
  issue_rows(P, w13_of<KIND>(L, g), s13_of<KIND>(L, g), 2 * L.I, L.H, ra, ra + 32);
  // One token: the dispatched position of a slot is the slot itself.
  BlockSumOut bs;
  if (KIND == kW8A8 && S.q8.gateup) {
    const int nb = L.H / kQBlock;
    bs.a = S.q8.gateup + ((size_t)slot * 2 * L.I + k) * nb;
    bs.b = S.q8.gateup + ((size_t)slot * 2 * L.I + L.I + k) * nb;
    bs.na = bs.nb = nb;
  }
  float r0, r1;
  dot_rows(P, L.H, sm.xl, sm.xq, sm.xs, r0, r1, bs);
  if ((lane & 15) == 0) S.gu[(size_t)slot * L.I + k] = silu(r0) * r1;
}

struct DownSmem {
  float hl[kMaxK + 2][kNarrow];
  int8_t hq[kMaxK + 2][kNarrow];
  float hs[kMaxK + 2][kNarrow / kQBlock];
  float yl[kMaxK + 2][8];
};

// Down: one workgroup per 8 output features; wave w < K = routed expert in
// ascending slot w, waves K and K+1 = the two halves of the shared expert's
// reduction (S/2 columns each); then the ordered combine of the 8 features:
// out = (residual +) ((y_s0 + y_s1) + p_0 y_0 + p_1 y_1 + ...), mul then add.
template <int KIND>
__global__ __launch_bounds__(64 * (kMaxK + 2)) void decode_down_kernel(DeviceLayer L, Scratch S,
                                                                       const float* residual,
                                                                       float* out) {
  __shared__ __align__(16) DownSmem sm;
  // Wave-uniform (scalar) so the per-wave buffer bases stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int f0 = 8 * blockIdx.x;
  const bool routed = wave < L.K;
  const int half = L.S / 2;
  // This wave's hidden row: an expert's I values, or half the shared S.
  const int n = routed ? L.I : half;
  const float* hrow = routed ? S.gu + (size_t)wave * L.I
                             : S.gu + (size_t)L.K * L.I + (size_t)(wave - L.K) * half;
  RowStage<kNarrow> Hr;
  load_row(Hr, hrow, n, lane);
  const int g = routed ? clamp_group(__builtin_amdgcn_readfirstlane(S.tiles[2 * wave]), L.E) : L.E;
  RowPair<KIND, kNarrow> P;
  issue_rows_cols(P, w2_of<KIND>(L, g), s2_of<KIND>(L, g), L.H, L.width(g),
                  routed ? 0 : (wave - L.K) * half, n, f0 + q, f0 + q + 4);
  // The combine inputs are loaded now and used last.
  float pw[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK; j++) pw[j] = j < L.K ? S.perm_w[j] : 0.0f;
  const float res_f = residual ? residual[f0 + (lane & 7)] : 0.0f;
  store_row(Hr, sm.hl[wave], n, lane);
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    quantize_lds(sm.hl[wave], n, sm.hq[wave], sm.hs[wave], lane, S.err);
    __syncthreads();
  }
  BlockSumOut bs;
  if (KIND == kW8A8 && (routed ? S.q8.down : S.q8.s_down)) {
    const int nb = L.width(g) / kQBlock;
    int32_t* row = routed ? S.q8.down + ((size_t)wave * L.H + f0 + q) * nb
                          : S.q8.s_down + (size_t)(f0 + q) * nb + (wave - L.K) * (half / kQBlock);
    bs.a = row;
    bs.b = row + (size_t)4 * nb;
    bs.na = bs.nb = n / kQBlock;
  }
  float r0, r1;
  dot_rows(P, n, sm.hl[wave], sm.hq[wave], sm.hs[wave], r0, r1, bs);
  if ((lane & 15) == 0) {
    sm.yl[wave][q] = r0;
    sm.yl[wave][q + 4] = r1;
  }
  __syncthreads();
  if (wave == 0 && lane < 8) {
    float acc = sm.yl[L.K][lane] + sm.yl[L.K + 1][lane];
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
    decode_gateup_kernel<KIND, KH>
        <<<dim3(L.S / kHidPerWg + L.K * (L.I / kHidPerWg)), dim3(64 * kUpWaves), 0, s>>>(L, S);
  else
    decode_down_kernel<KIND><<<dim3(L.H / 8), dim3(64 * (L.K + 2)), 0, s>>>(L, S, residual, out);
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
  // Gate/up rows reduce over H (<= 2048), 32 hidden values per workgroup;
  // the down launch reduces over I (<= 1024, one wave per routed expert) and
  // the two halves of S (<= 2048, each a whole number of 32-blocks);
  // routing is one wave over E <= 64 logits.
  return L.H <= kWide && L.S <= kWide && L.I <= kNarrow && L.K >= 1 && L.K <= kMaxK &&
         L.E <= 64 && L.H % 8 == 0 && L.I % kHidPerWg == 0 && L.S % kHidPerWg == 0 &&
         L.S % 64 == 0;
}

void launch_decode_stage(int stage, const DeviceLayer& L, const Scratch& S, const float* residual,
                         float* out, hipStream_t s) {
  if (L.H <= 1280)
    launch_kind<1280>(stage, L, S, residual, out, s);
  else
    launch_kind<kWide>(stage, L, S, residual, out, s);
}

}  // namespace uocr
