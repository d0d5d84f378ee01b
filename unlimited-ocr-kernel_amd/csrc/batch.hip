// Small-batch expert engine: row tiles of up to 16 tokens of one expert
// group (the shared expert is group E). A workgroup takes one slice of one
// tile's weight rows (a unit), issues every load of the slice at once and
// dots it with the tile's activation rows staged in LDS. The grid is one
// unit per workgroup, shared-expert units first (they need nothing from
// the dispatch), then the slices of each routed tile; workgroups are kept
// small (19 KiB of LDS, <= 128 or 168 VGPRs) so that several share a CU and
// their chains of dependent loads overlap. Used for 2 <= T <= 16, and for
// the single-row W8A8 groups of INT8 layers at any T. In INT8 weight-only
// layers the shared expert's units run as MFMA tiles of 16 tokens instead
// (the routed units keep the dot).
//
// Also the fence-free small-batch router (2 <= T <= 16): one launch whose
// logit workgroups count themselves in; the last one routes every token
// and builds the dispatch. In INT8 weight-only layers its launch also runs
// the shared expert's gate/up units.
//
// Arithmetic: Decoder::projection / feed_forward (src/decoder/mod.rs:
// 99-122) per row; INT8 weight-only as q * x summed per 16-byte chunk and
// scaled by the chunk's block scale (MFMA units: per 32-block, with the
// activations as bf16 hi + lo parts); W8A8 only for DynamicActivations
// groups of a single row (:103-104).
#include <type_traits>

#include "common.hpp"
#include "moe_kernels.hpp"
#include "routing.hpp"
#include "rowdot.hpp"

namespace uocr {

namespace {

constexpr int kTileRows = kGemvChunk;  // tokens per row tile
constexpr int kDotTok = 4;             // tokens per register batch of the dot
// FP32 activations staged per workgroup (16 KiB: three 1280-wide rows per
// pass). 36 KiB (seven rows) allowed four workgroups per CU; at 16 KiB the
// VGPRs set the limit, and the 16-token INT8 forward went 76.7 -> 75.3 us.
constexpr int kStage = 4096;
constexpr int kWideK = 2048;           // widest reduction dimension (H, S)
constexpr int kSegK = 1024;            // widest down-projection segment in registers
// Shared-expert tiles take 8 rows: their units dot every weight with each
// row, and at 16 rows they were the longest units of a launch.
constexpr int kSharedRows = 8;

// Workgroups of 256 threads per CU: four (at most 128 VGPRs per lane) for
// the gate/up GEMV where INT8 rows of up to 1280 bytes fit, three (168)
// otherwise. The down GEMV measured faster at three (its staged activation
// rows are longer and its shared-expert units heavier).
template <int KIND, int KMAX, bool DYN>
constexpr int batch_waves() {
  return !DYN && KIND == kInt8 && KMAX <= 1280 ? 4 : 3;
}

// Down-projection rows of a group of width W: full rows (32 per unit) up to
// kSegK, otherwise two column halves of seg_of(W) per row (16 rows per unit).
__host__ __device__ inline int seg_of(int W) {
  return W <= kSegK ? W : ((W + 1) / 2 + kQBlock - 1) / kQBlock * kQBlock;
}
__host__ __device__ inline int down_units(int H, int W) { return W <= kSegK ? H / 32 : H / 16; }

struct Unit {
  int g, r0, n, group_rows, slice;
  bool routed;
  int base;          // first dispatched position (routed) or row (shared); < 0: read the offsets
  const int* rows;   // the tile's tokens from its record (null: the permutation)
};

// Routed unit b: ur slices of each routed tile of the dispatch list. With
// the small router's tile records, one load gives the group, its position
// and rows, and the tokens (record i is written for every listed tile, and
// i stays inside the records' allocation).
__device__ __forceinline__ bool routed_unit(const Scratch& S, int mchunk, int ur, int b, Unit& u) {
  const int i = b / ur;
  u.routed = true;
  u.slice = b - i * ur;
  if (S.tile_desc) {
    const int* d = S.tile_desc + (size_t)i * kTileDescInts;
    const int routed_tiles = S.counters[1];
    const int g = d[0], base = d[1], rows = d[2];
    if (i >= routed_tiles) return false;
    u.g = g;
    u.r0 = 0;
    u.base = base;
    u.rows = d + 4;
    u.group_rows = rows;
    u.n = min(mchunk, rows);
    return u.n > 0;
  }
  // Both loads in flight together; i stays inside the list's allocation.
  const int routed_tiles = S.counters[1];
  const int g = S.tiles[2 * i], r0 = S.tiles[2 * i + 1];
  if (i >= routed_tiles) return false;
  u.g = g;
  u.r0 = r0;
  const int first = S.offsets[g];
  u.group_rows = S.offsets[g + 1] - first;
  u.base = first + r0;
  u.rows = nullptr;
  u.n = min(mchunk, u.group_rows - r0);
  return u.n > 0;
}

// Unit blockIdx.x: the nsh shared tiles' us slices each come first (tile ts
// holds rows [ts * kSharedRows, ...) of the shared group), then the routed
// units.
__device__ __forceinline__ bool load_unit(const DeviceLayer& L, const Scratch& S, int T, int mchunk,
                                          int nsh, int us, int ur, Unit& u) {
  const int b = blockIdx.x;
  if (b < nsh * us) {
    const int ts = b / us;
    u.g = L.E;
    u.routed = false;
    u.r0 = ts * kSharedRows;
    u.base = u.r0;
    u.rows = nullptr;
    u.slice = b - ts * us;
    u.group_rows = T;
    u.n = min(kSharedRows, T - u.r0);
    return u.n > 0;
  }
  return routed_unit(S, mchunk, ur, b - nsh * us, u);
}

// The single-row pass (the W8A8 rows the MFMA engine leaves to this engine
// under DynamicActivations): kernels of their own, whose workgroups each
// read the expert offsets once and loop over the units of the groups of
// exactly one row, so that a pass with no such group is one short round.
// Routed groups of one row as a mask over expert ids (E <= 64).
__device__ __forceinline__ unsigned long long single_groups(const DeviceLayer& L,
                                                           const Scratch& S) {
  const int e = threadIdx.x & 63;
  const bool one = e < L.E && S.offsets[e + 1] - S.offsets[e] == 1;
  return __ballot(one);
}

// Unit b of those groups' units (ur per group, ascending expert id), for
// b < popcount(m) * ur. Every lane of the wave takes part.
__device__ __forceinline__ Unit single_unit(unsigned long long m, int ur, int b) {
  const int lane = threadIdx.x & 63;
  const int j = b / ur;
  const bool hit = ((m >> lane) & 1ull) && __popcll(m & ((1ull << lane) - 1ull)) == j;
  Unit u;
  u.g = __ffsll((long long)__ballot(hit)) - 1;
  u.r0 = 0;
  u.n = 1;
  u.group_rows = 1;
  u.routed = true;
  u.base = -1;
  u.rows = nullptr;
  u.slice = b - j * ur;
  return u;
}

// Workgroups of a single-row pass: three per CU, one round.
constexpr int kSinglesGrid = 768;

// Row of w13 holding gate value k (up value k is 32 rows further).
__device__ __forceinline__ int gate_row(int k) { return (k >> 5) * 64 + (k & 31); }

struct BatchSmem {
  float x[kStage];
  int8_t xq[kWideK];
  float xs[kWideK / kQBlock];
  const float* rows[kTileRows];
};

// Stages activation rows [b0, b0 + nb) of the tile into LDS at stride ld
// (columns [K, ld) zero) with every thread; `row_of(t)` gives the source
// row pointer. K and ld are multiples of 4.
template <typename RowOf>
__device__ __forceinline__ void stage_tile(BatchSmem& sm, int b0, int nb, int K, int ld,
                                           RowOf row_of) {
  if (threadIdx.x < nb) sm.rows[threadIdx.x] = row_of(b0 + threadIdx.x);
  __syncthreads();
  const int vec = ld / 4, kvec = K / 4;
  const int total = nb * vec;
  constexpr int kPer = 4;
  for (int base = 0; base < total; base += kPer * 256) {
    u32x4 v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int at = base + threadIdx.x + i * 256;
      const int t = at / vec, c = at - t * vec;
      v[i] = u32x4{0u, 0u, 0u, 0u};
      if (at < total && c < kvec) v[i] = reinterpret_cast<const u32x4*>(sm.rows[t])[c];
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

// Dots the loaded row segments (K columns each; the b segment from column
// XB of the staged row) with the tile's activations in token batches that
// fit the LDS budget; emit(t, r0, r1) receives every token's two segment
// sums (in every lane of the row's 16-lane group). K valid columns of each
// activation row are staged at stride ld (zero beyond). A single-row tile
// of an INT8 layer in DynamicActivations mode takes the W8A8 dot instead.
// `sums`: where the W8A8 dot stores its block sums (a test trace).
template <int KIND, int KMAX, int XB, bool DYN, typename RowOf, typename Emit>
__device__ __forceinline__ void tile_dot(const DeviceLayer& L, const Scratch& S, BatchSmem& sm,
                                         const RowPair<KIND, KMAX>& P, int K, int xb, int cols,
                                         int ld, const Unit& u, RowOf row_of, Emit emit,
                                         const BlockSumOut& sums = BlockSumOut()) {
  const int lane = threadIdx.x & 63;
  const int xb_off = XB ? xb : 0;
  if constexpr (KIND == kInt8 && DYN) {
    if (u.group_rows == 1) {
      stage_tile(sm, 0, 1, cols, ld, row_of);
      // The zero columns quantise to zero blocks, so every block a segment
      // can reach is defined.
      quantize_lds_waves(sm.x, ld, sm.xq, sm.xs, threadIdx.x >> 6, blockDim.x >> 6, lane, S.err);
      __syncthreads();
      float r0, r1;
      dot_rows_as<kW8A8>(P, K, sm.x, sm.xq, sm.xs, r0, r1, xb_off, sums);
      emit(0, r0, r1);
      return;
    }
  }
  // Tokens staged per pass (LDS budget), dotted kDotTok at a time; the
  // weight rows stay in registers throughout.
  const int per = kStage / ld < kTileRows ? kStage / ld : kTileRows;
  for (int b0 = 0; b0 < u.n; b0 += per) {
    const int nb = min(per, u.n - b0);
    if (b0 > 0) __syncthreads();  // the previous pass is consumed
    stage_tile(sm, b0, nb, cols, ld, row_of);
    for (int d0 = 0; d0 < nb; d0 += kDotTok) {
      auto run = [&](auto ntc) {
        constexpr int NT = decltype(ntc)::value;
        float a0[NT], a1[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) a0[t] = a1[t] = 0.0f;
        dot_rows_multi<KIND, KMAX, NT, XB != 0>(P, K, sm.x + d0 * ld, xb_off, ld, a0, a1);
#pragma unroll
        for (int t = 0; t < NT; t++) emit(b0 + d0 + t, row16_sum(a0[t]), row16_sum(a1[t]));
      };
      static_assert(kDotTok == 4, "one case per batch size");
      switch (min(kDotTok, nb - d0)) {
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        case 3: run(std::integral_constant<int, 3>{}); break;
        default: run(std::integral_constant<int, 4>{}); break;
      }
    }
  }
}

// Gate/up: a unit is 16 hidden values of one tile (each wave 4 gate rows
// and the 4 matching up rows). h = silu(gate) * up (Decoder::feed_forward,
// src/decoder/mod.rs:114-122).
// SINGLE: the single-row pass beside the MFMA engine, whose hidden row of
// the group at dispatched position p lives at gu + p I (the MFMA engine's
// hidden planes take the bytes of h; p < T K, so the T K rows of I floats
// fit gu whatever the expert ids); the W8A8 trace's hidden row is then
// written here, so the trace's positions of multi-row groups stay untouched.
template <int KIND, int KH, bool DYN, bool SINGLE = false>
__device__ __forceinline__ void gateup_body(const DeviceLayer& L, const Scratch& S, BatchSmem& sm,
                                            const Unit& u) {
  const int W = L.width(u.g);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = 16 * u.slice + 4 * wave + (lane >> 4);
  const int ra = gate_row(k);
  RowPair<KIND, KH> P;
  issue_rows(P, w13_of<KIND>(L, u.g), s13_of<KIND>(L, u.g), 2 * W, L.H, ra, ra + 32);
  const int base = u.base >= 0 ? u.base : S.offsets[u.g] + u.r0;
  auto row_of = [&](int t) {
    const int row = u.rows ? u.rows[t] : u.routed ? S.perm_rows[base + t] : base + t;
    return S.xn + (size_t)row * L.H;
  };
  float* hout = SINGLE     ? S.gu + (size_t)base * L.I
                : u.routed ? S.h + (size_t)base * L.I
                           : S.hs + (size_t)base * L.S;
  const int ld = u.routed ? L.I : L.S;
  // The W8A8 trace's hidden row of a single-row group (routed: position
  // base; the shared expert, a single row only at T = 1: its own row).
  float* htrace = nullptr;
  if (DYN && u.group_rows == 1)
    htrace = !u.routed ? S.q8.s_hidden : S.q8.hidden ? S.q8.hidden + (size_t)base * L.I : nullptr;
  BlockSumOut bs;
  if (DYN && u.group_rows == 1 && k < W) {
    // A single-row group: position `base` (routed) or the one token (shared).
    const int nb = L.H / kQBlock;
    int32_t* at = u.routed ? (S.q8.gateup ? S.q8.gateup + (size_t)base * 2 * L.I * nb : nullptr)
                           : S.q8.s_gateup;
    if (at) {
      bs.a = at + (size_t)k * nb;
      bs.b = at + (size_t)(W + k) * nb;
      bs.na = bs.nb = nb;
    }
  }
  tile_dot<KIND, KH, 0, DYN>(L, S, sm, P, L.H, 0, L.H, L.H, u, row_of, [&](int t, float g, float up) {
    if ((lane & 15) == 0 && k < W) {
      const float h = silu(g) * up;
      hout[(size_t)t * ld + k] = h;
      if (htrace) htrace[k] = h;
    }
  }, bs);
}

template <int KIND, int KH, bool DYN>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(batch_waves<KIND, KH, DYN>()))) void batch_gateup_kernel(
    DeviceLayer L, Scratch S, int T, int mchunk, int nsh) {
  __shared__ __align__(16) BatchSmem sm;
  Unit u;
  if (!load_unit(L, S, T, mchunk, nsh, (L.S + 15) / 16, (L.I + 15) / 16, u)) return;
  gateup_body<KIND, KH, DYN>(L, S, sm, u);
}

// Gate/up of the single-row W8A8 groups (INT8 weights, DynamicActivations).
// Hidden widths beyond 1280 take two workgroups per CU (their loop spilled
// at three).
template <int KH>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(KH <= 1280 ? 3 : 2))) void singles_gateup_kernel(
    DeviceLayer L, Scratch S) {
  __shared__ __align__(16) BatchSmem sm;
  const unsigned long long m = single_groups(L, S);
  const int ur = (L.I + 15) / 16, n = __popcll(m) * ur;
  for (int b = blockIdx.x; b < n; b += gridDim.x) {
    gateup_body<kInt8, KH, true, true>(L, S, sm, single_unit(m, ur, b));
    __syncthreads();  // this unit's LDS consumed before the next is staged
  }
}

// Down: a unit is 32 output features of one tile (each wave 8 full rows of
// the down matrix), or, for widths beyond kSegK, 16 output features with
// each row's two column halves in the lanes' two segments. Writes y
// (routed, dispatched order) or ys.
template <int KIND, bool HALVES, bool DYN, bool SINGLE = false>
__device__ __forceinline__ void down_body(const DeviceLayer& L, const Scratch& S, BatchSmem& sm,
                                          const Unit& u) {
  const int W = L.width(u.g);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int seg = seg_of(W);
  const int ra = HALVES ? 16 * u.slice + 4 * wave + (lane >> 4) : 32 * u.slice + 8 * wave + (lane >> 4);
  const int rb = HALVES ? ra : ra + 4;
  RowPair<KIND, kSegK> P;
  issue_segs(P, w2_of<KIND>(L, u.g), s2_of<KIND>(L, u.g), L.H, W, ra, 0, rb, HALVES ? seg : 0, seg);
  const int base = u.base >= 0 ? u.base : S.offsets[u.g] + u.r0;
  const float* hin = SINGLE     ? S.gu + (size_t)base * L.I
                      : u.routed ? S.h + (size_t)base * L.I
                                 : S.hs + (size_t)base * L.S;
  auto row_of = [&](int t) { return hin + (size_t)t * W; };
  float* yout = u.routed ? S.y + (size_t)base * L.H : S.ys + (size_t)base * L.H;
  BlockSumOut bs;
  if (DYN && u.group_rows == 1) {
    // Rows [H][W/32] of a single-row group's down projection: full rows ra
    // and rb, or the two column halves of row ra.
    const int nb = W / kQBlock;
    int32_t* at = u.routed ? (S.q8.down ? S.q8.down + (size_t)base * L.H * nb : nullptr) : S.q8.s_down;
    if (at && ra < L.H) {
      bs.a = at + (size_t)ra * nb;
      if (HALVES) {
        bs.b = bs.a + seg / kQBlock;
        bs.na = seg / kQBlock;
        bs.nb = nb - seg / kQBlock;
      } else {
        bs.b = rb < L.H ? at + (size_t)rb * nb : nullptr;
        bs.na = bs.nb = nb;
      }
    }
  }
  tile_dot<KIND, kSegK, HALVES ? 1 : 0, DYN>(L, S, sm, P, seg, seg, W, HALVES ? 2 * seg : W, u, row_of,
                                        [&](int t, float y0, float y1) {
    if ((lane & 15) == 0) {
      if (HALVES) {
        if (ra < L.H) yout[(size_t)t * L.H + ra] = y0 + y1;
      } else {
        if (ra < L.H) yout[(size_t)t * L.H + ra] = y0;
        if (rb < L.H) yout[(size_t)t * L.H + rb] = y1;
      }
    }
  }, bs);
}

template <int KIND, bool DYN>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(3))) void batch_down_kernel(
    DeviceLayer L, Scratch S, int T, int mchunk, int nsh) {
  __shared__ __align__(16) BatchSmem sm;
  Unit u;
  if (!load_unit(L, S, T, mchunk, nsh, down_units(L.H, L.S), down_units(L.H, L.I), u))
    return;
  if (L.width(u.g) <= kSegK)
    down_body<KIND, false, DYN>(L, S, sm, u);
  else
    down_body<KIND, true, DYN>(L, S, sm, u);
}

// MFMA form of the shared expert's units: a tile of up to 16 tokens times
// one or two sets of 16 weight rows (gate and up rows of 16 hidden values,
// or 16 or 32 down rows), as v_mfma_f32_16x16x32_bf16 products. A = the
// tokens' activations as bf16 hi and lo parts (FP32-class: the input rows
// split as they are loaded, the hidden rows handed over as k-blocked
// [K/32][rows][32] planes); B = 16 rows of one 32-block from the k-blocked
// panels: BF16 weights as stored, or INT8 rows widened to bf16 (exact),
// whose per-block partial is folded into the accumulator with the rows'
// block scales (Decoder::projection, src/decoder/mod.rs:99-112, with the
// scale applied per 32-block; under DynamicActivations the shared group
// of T >= 2 rows is weight-only, :103-104). Wave w of the unit's four
// takes the w-th quarter of the blocks; the four partial tiles meet in
// LDS, summed in wave order. The MFMA costs the same for 1 or 16 tokens,
// so the shared tiles take 16 rows; routed tiles (about two tokens each)
// stay on the dot, where a 16-row A operand's loads cost more than the
// MFMA saves (the 16-token INT8 forward's gate/up launch took 50.7 instead
// of 35.2 us with every unit in MFMA form).
//
// Where they run (2 <= T <= 16, hidden width <= 1280): the shared gate/up
// units in the router's launch, beside its logit workgroups (they need no
// routing), and the shared down units at the head of the gate/up launch;
// the down launch then holds routed units only. Otherwise (INT8 layers
// only) the shared units head the gate/up and down launches.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kMfmaSharedRows = 16;
constexpr int kMfmaWaves = 4;
constexpr int kPartLd = 20;  // floats per row of a partial tile (16 tokens + pad, 16-byte aligned)

struct MfmaUnitSmem {
  float part[kMfmaWaves][2][16][kPartLd];  // [wave][row set][row][token]
};
union SharedSmem {
  BatchSmem b;
  MfmaUnitSmem m;
};

// Eight int8 weights as bf16 (the f32 of a small integer has a zero low
// half, so its bf16 is the high half).
__device__ __forceinline__ bf16x8 widen_q8(u32x2 q) {
  uint32_t hp[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t word = j < 2 ? q.x : q.y;
    const int s0 = 16 * (j & 1);
    const float w0 = (float)(int8_t)((word >> s0) & 0xffu);
    const float w1 = (float)(int8_t)((word >> (s0 + 8)) & 0xffu);
    hp[j] = __builtin_amdgcn_perm(__float_as_uint(w1), __float_as_uint(w0), 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8, u32x4{hp[0], hp[1], hp[2], hp[3]});
}

// Rows ra (and, with NSET = 2, rb) -- this lane's column of each row set --
// of a k-blocked panel [K/32][rows][32] (BF16, or INT8 with row-major block
// scales [rows][K/32]), dotted with activation row xrow: with F32X, FP32
// rows [prows][K] split into bf16 hi and lo parts here; otherwise bf16
// planes (hi at `act`, lo prows * K elements later, k-blocked
// [K/32][prows][32]). acc_a / acc_b hold this wave's blocks' sums for tokens
// 4 (lane / 16) .. + 3. Rows outside [0, rows) read as zero. Lanes are
// numbered within the unit's four waves (threadIdx.x mod 256).
template <int KIND, int KMAX, int NSET, bool F32X>
__device__ __forceinline__ void mfma_rows_dot(const void* panel, const float* scales, int rows,
                                              int K, int ra, int rb, const void* act, int prows,
                                              int xrow, f32x4& acc_a, f32x4& acc_b) {
  constexpr bool kQ8 = KIND == kInt8;
  const int wave = (threadIdx.x >> 6) & 3, grp = (threadIdx.x >> 4) & 3;
  const int nblk = K / kQBlock;
  constexpr int kBW = KMAX / kQBlock / kMfmaWaves;  // blocks per wave, at most
  constexpr int kB2 = NSET == 2 ? kBW : 1;
  constexpr uint32_t kRowB = kQ8 ? 32u : 64u;       // bytes per row and block
  const int per = (nblk + kMfmaWaves - 1) / kMfmaWaves;
  const int kb0 = wave * per;
  // Weights (and scales) first: they need only the group.
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(panel, (uint32_t)rows * (uint32_t)K * (kRowB / 32u));
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(kQ8 ? (const void*)scales : panel, kQ8 ? (uint32_t)rows * (uint32_t)nblk * 4u : 0u);
  u32x2 qa[kQ8 ? kBW : 1], qb[kQ8 ? kB2 : 1];
  u32x4 ha[kQ8 ? 1 : kBW], hb[kQ8 ? 1 : kB2];
  float sa[kQ8 ? kBW : 1], sb[kQ8 ? kB2 : 1];
#pragma unroll
  for (int i = 0; i < kBW; i++) {
    const int kb = kb0 + i;
    const bool ok = i < per && kb < nblk;
    const uint32_t at = (uint32_t)kb * rows;
    const uint32_t oa = ok && ra < rows ? (at + ra) * kRowB + (kRowB / 4u) * grp : kOut;
    const uint32_t ob = ok && rb < rows ? (at + rb) * kRowB + (kRowB / 4u) * grp : kOut;
    if constexpr (kQ8) {
      qa[i] = __builtin_amdgcn_raw_buffer_load_b64(wr, oa, 0, 0);
      sa[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          sr, ok && ra < rows ? ((uint32_t)ra * nblk + kb) * 4u : kOut, 0, 0));
      if constexpr (NSET == 2) {
        qb[i] = __builtin_amdgcn_raw_buffer_load_b64(wr, ob, 0, 0);
        sb[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            sr, ok && rb < rows ? ((uint32_t)rb * nblk + kb) * 4u : kOut, 0, 0));
      }
    } else {
      ha[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, oa, 0, 0);
      if constexpr (NSET == 2) hb[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, ob, 0, 0);
    }
  }
  const uint32_t plane = (uint32_t)prows * (uint32_t)K;  // elements per plane or per row set
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(act, plane * 4u);
  acc_a = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  acc_b = acc_a;
#pragma unroll
  for (int i = 0; i < kBW; i++) {
    const int kb = kb0 + i;
    const bool ok = i < per && kb < nblk;
    bf16x8 xh, xl;
    if constexpr (F32X) {
      const uint32_t at = ((uint32_t)xrow * K + (uint32_t)kb * 32u + 8u * grp) * 4u;
      const u32x4 f0 = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? at : kOut, 0, 0);
      const u32x4 f1 = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? at + 16u : kOut, 0, 0);
      const uint32_t f[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float a = __uint_as_float(f[2 * j]), b = __uint_as_float(f[2 * j + 1]);
        h[j] = bf16_pair(a, b);
        l[j] = bf16_pair(a - bf16_lo(h[j]), b - bf16_hi(h[j]));
      }
      xh = __builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]});
      xl = __builtin_bit_cast(bf16x8, u32x4{l[0], l[1], l[2], l[3]});
    } else {
      const uint32_t at = ((uint32_t)kb * prows + xrow) * 64u + 16u * grp;
      xh = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? at : kOut, 0, 0));
      xl = __builtin_bit_cast(
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? at + plane * 2u : kOut, 0, 0));
    }
    if constexpr (kQ8) {
      const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
      const bf16x8 wa = widen_q8(qa[i]);
      f32x4 pa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wa, z, 0, 0, 0);
      pa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wa, pa, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; r++) acc_a[r] = __builtin_fmaf(pa[r], sa[i], acc_a[r]);
      if constexpr (NSET == 2) {
        const bf16x8 wb = widen_q8(qb[i]);
        f32x4 pb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wb, z, 0, 0, 0);
        pb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wb, pb, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) acc_b[r] = __builtin_fmaf(pb[r], sb[i], acc_b[r]);
      }
    } else {
      const bf16x8 wa = __builtin_bit_cast(bf16x8, ha[i]);
      acc_a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wa, acc_a, 0, 0, 0);
      acc_a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wa, acc_a, 0, 0, 0);
      if constexpr (NSET == 2) {
        const bf16x8 wb = __builtin_bit_cast(bf16x8, hb[i]);
        acc_b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wb, acc_b, 0, 0, 0);
        acc_b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wb, acc_b, 0, 0, 0);
      }
    }
  }
}

// Sums the unit's four waves' partial tiles in wave order (one barrier for
// the whole workgroup): thread (c = tid % 16, t = tid / 16 % 16) receives
// row c of each set for token t.
__device__ __forceinline__ void mfma_reduce(MfmaUnitSmem& sm, const f32x4& acc_a,
                                            const f32x4& acc_b, float& a, float& b) {
  const int wave = (threadIdx.x >> 6) & 3, col = threadIdx.x & 15, grp = (threadIdx.x >> 4) & 3;
  *reinterpret_cast<f32x4*>(&sm.part[wave][0][col][4 * grp]) = acc_a;
  *reinterpret_cast<f32x4*>(&sm.part[wave][1][col][4 * grp]) = acc_b;
  __syncthreads();
  const int c = threadIdx.x & 15, t = (threadIdx.x >> 4) & 15;
  a = sm.part[0][0][c][t];
  b = sm.part[0][1][c][t];
#pragma unroll
  for (int w = 1; w < kMfmaWaves; w++) {
    a += sm.part[w][0][c][t];
    b += sm.part[w][1][c][t];
  }
}

// bf16 planes of the shared expert's hidden rows ([S/32][T][32], hi then
// lo), in bytes the small-batch engine leaves free.
__device__ __forceinline__ uint16_t* shared_hidden_planes(const Scratch& S) {
  return reinterpret_cast<uint16_t*>(S.gu);
}

// Shared gate/up unit: hidden values 16 slice .. + 15 for tokens [r0, r0 + n)
// of the input rows; h = silu(gate) * up (src/decoder/mod.rs:114-122) goes
// to the hidden planes. A unit that is not `live` still takes part in the
// workgroup's barrier and stores nothing.
template <int KIND, int KH>
__device__ __forceinline__ void shared_gateup_mfma(const DeviceLayer& L, const Scratch& S,
                                                   MfmaUnitSmem& sm, int slice, int r0, int n,
                                                   int T, bool live) {
  const int W = L.S, col = threadIdx.x & 15;
  const int k0 = 16 * slice;
  const int ra = live ? gate_row(k0) + col : 2 * W;
  f32x4 ag, au;
  const void* panel = KIND == kInt8 ? (const void*)(L.q13k + L.w13_offset(L.E))
                                    : (const void*)(L.w13k + L.w13_offset(L.E));
  mfma_rows_dot<KIND, KH, 2, true>(panel, KIND == kInt8 ? L.s13 + L.s13_offset(L.E) : nullptr,
                                   2 * W, L.H, ra, ra + 32, S.xn, T, r0 + min(col, n - 1), ag, au);
  float g, up;
  mfma_reduce(sm, ag, au, g, up);
  const int c = threadIdx.x & 15, t = (threadIdx.x >> 4) & 15, k = k0 + c;
  if (live && t < n && k < W) {
    const float h = silu(g) * up;
    const uint16_t hb = __builtin_bit_cast(uint16_t, (__bf16)h);
    const uint16_t lb = __builtin_bit_cast(uint16_t, (__bf16)(h - __uint_as_float((uint32_t)hb << 16)));
    uint16_t* hp = shared_hidden_planes(S);
    const size_t p = ((size_t)(k / 32) * T + r0 + t) * 32 + k % 32;
    hp[p] = hb;
    hp[(size_t)T * W + p] = lb;
  }
}

// Shared down unit: output features 16 NSET slice .. for tokens [r0, r0 + n).
template <int KIND, int NSET>
__device__ __forceinline__ void shared_down_mfma(const DeviceLayer& L, const Scratch& S,
                                                 MfmaUnitSmem& sm, int slice, int r0, int n, int T) {
  const int W = L.S, col = threadIdx.x & 15;
  const int n0 = 16 * NSET * slice;
  f32x4 aa, ab;
  const void* panel = KIND == kInt8 ? (const void*)(L.q2k + L.w2_offset(L.E))
                                    : (const void*)(L.w2k + L.w2_offset(L.E));
  mfma_rows_dot<KIND, kWideK, NSET, false>(panel, KIND == kInt8 ? L.s2 + L.s2_offset(L.E) : nullptr,
                                           L.H, W, n0 + col, n0 + 16 + col,
                                           shared_hidden_planes(S), T, r0 + min(col, n - 1), aa, ab);
  float ya, yb;
  mfma_reduce(sm, aa, ab, ya, yb);
  const int c = threadIdx.x & 15, t = (threadIdx.x >> 4) & 15;
  if (t < n) {
    float* yout = S.ys + (size_t)(r0 + t) * L.H;
    if (n0 + c < L.H) yout[n0 + c] = ya;
    if (NSET == 2 && n0 + 16 + c < L.H) yout[n0 + 16 + c] = yb;
  }
}

// Whether the shared expert's units take the MFMA form: weight-only math
// on its group (not the single-row W8A8 group of a one-token forward under
// DynamicActivations). BF16 weights: up to 1280 hidden values and 16
// tokens (their two-set down units would not fit the registers beyond);
// DynamicActivations: up to 1280 hidden values (the wider W8A8 gate/up
// kernel has no registers to spare).
__host__ __device__ inline bool mfma_shared(const DeviceLayer& L, int T) {
  if (L.S <= 0 || L.S % 32 != 0) return false;
  if (L.quant_mode == kQuantWeightsOnly) return true;
  if (L.quant_mode == kQuantNone) return L.H <= 1280 && T <= kTileRows;
  return L.H <= 1280 && T >= 2;  // DynamicActivations
}

// Whether the router's launch runs the shared gate/up units (then the
// gate/up launch runs the shared down units, 16 rows each).
__host__ __device__ inline bool shared_in_router(const DeviceLayer& L, int T) {
  return mfma_shared(L, T) && L.H <= 1280 && T <= kTileRows;
}

// Gate/up launch with MFMA shared units: sdn shared down units (16 rows of
// the one shared tile), then sgu shared gate/up units (16-token tiles,
// (S + 15) / 16 per tile), then the routed units on the dot.
template <int KIND, int KH, bool DYN>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(batch_waves<KIND, KH, DYN>()))) void batch_gateup_ms_kernel(
    DeviceLayer L, Scratch S, int T, int mchunk, int sdn, int sgu) {
  __shared__ __align__(16) SharedSmem sm;
  int b = blockIdx.x;
  if (b < sdn) {
    shared_down_mfma<KIND, 1>(L, S, sm.m, b, 0, T, T);
    return;
  }
  b -= sdn;
  if (b < sgu) {
    const int us = (L.S + 15) / 16, ts = b / us;
    const int r0 = ts * kMfmaSharedRows;
    shared_gateup_mfma<KIND, KH>(L, S, sm.m, b - ts * us, r0, min(kMfmaSharedRows, T - r0), T, true);
    return;
  }
  Unit u;
  if (routed_unit(S, mchunk, (L.I + 15) / 16, b - sgu, u)) gateup_body<KIND, KH, DYN>(L, S, sm.b, u);
}

// Down launch with MFMA shared units: sdn shared down units (32 rows of one
// 16-token tile; INT8 only), then the routed units on the dot.
template <int KIND, bool DYN>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(3))) void batch_down_ms_kernel(DeviceLayer L, Scratch S, int T,
                                                                 int mchunk, int sdn) {
  __shared__ __align__(16) SharedSmem sm;
  const int b = blockIdx.x;
  if constexpr (KIND == kInt8) {
    if (b < sdn) {
      const int us = L.H / 32, ts = b / us;
      const int r0 = ts * kMfmaSharedRows;
      shared_down_mfma<KIND, 2>(L, S, sm.m, b - ts * us, r0, min(kMfmaSharedRows, T - r0), T);
      return;
    }
  }
  Unit u;
  if (!routed_unit(S, mchunk, down_units(L.H, L.I), b - sdn, u)) return;
  if (L.I <= kSegK)
    down_body<KIND, false, DYN>(L, S, sm.b, u);
  else
    down_body<KIND, true, DYN>(L, S, sm.b, u);
}

// Down of the single-row W8A8 groups; HALVES as down_body (routed width
// beyond kSegK).
template <bool HALVES>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(3))) void singles_down_kernel(DeviceLayer L, Scratch S) {
  __shared__ __align__(16) BatchSmem sm;
  const unsigned long long m = single_groups(L, S);
  const int ur = down_units(L.H, L.I), n = __popcll(m) * ur;
  for (int b = blockIdx.x; b < n; b += gridDim.x) {
    down_body<kInt8, HALVES, true, true>(L, S, sm, single_unit(m, ur, b));
    __syncthreads();  // this unit's LDS consumed before the next is staged
  }
}

// ------------------------------------------------------------- small router

// Routing of T <= 16 tokens in one launch. Workgroup (b, p) dots router
// rows 8b .. 8b+7 with tokens 2p, 2p+1 on its first two waves (so the 2·H·E·T
// flops spread over E/8 · T/2 workgroups, and the router rows come from L2
// after the first touch) and stores the logits device-coherently. Once its
// stores are complete it counts itself in one of 8 sub-counts (workgroup
// id mod 8); the one completing a sub-count counts that in a top count and
// zeroes the sub-count; the one completing the top count zeroes it and,
// with all 16 waves, routes and dispatches every token, reading the logits
// device-coherently (no word takes more than 8 counts). Wave t routes token
// t (moe::route, src/decoder/moe.rs:7-30), then the dispatch of
// Decoder::experts (src/decoder/mod.rs:127-141): per expert, its tokens in
// ascending order; one row tile per active expert and one for the shared
// expert.
constexpr int kRouterTok = 2;
constexpr int kRouteWaves = 16;

__device__ __forceinline__ void route_dispatch(const DeviceLayer& L, const Scratch& S, int T,
                                               int wave, int lane) {
  __shared__ unsigned long long masks[kRouteWaves];
  __shared__ unsigned long long active_mask;
  __shared__ int count[64];
  __shared__ int start[65];
  const int E = L.E, K = L.K;
  const bool mine = wave < T;
  // Waves past T route a neutral row (their result is not used).
  const float v = mine && lane < E ? __hip_atomic_load(S.logits + (size_t)wave * E + lane,
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : 0.0f;
  const WaveSel r = route_wave_sel(v, E, K);
  const float w = route_weight(r, L.normalize, L.scale);
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
    const unsigned long long am = __ballot(count[lane] > 0);
    if (lane == 0) active_mask = am;
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
    if (S.tile_desc) {
      // The token's place in its group's record (one tile per active group).
      const int slot = __popcll(active_mask & ((1ull << lane) - 1ull));
      S.tile_desc[(size_t)slot * kTileDescInts + 4 + before] = wave;
    }
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
      if (S.tile_desc) {
        int* d = S.tile_desc + (size_t)slot * kTileDescInts;
        d[0] = lane;
        d[1] = start[lane];
        d[2] = count[lane];
      }
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

// Workgroups [0, n_route): router column b = id % ceil(E / 8) (rows 8b ..
// 8b + 7) for tokens 2p, 2p + 1 (p = id / ceil(E / 8)). Each workgroup from
// n_route on runs one of the shared expert's gate/up units on its first
// four waves (they need no routing and take no part in the count); one
// unit per workgroup, so that the units' weight streams spread over as
// many CUs (with four units per 16-wave workgroup, 28 CUs streamed the
// shared rows and the launch took 22.8 instead of 8.9 us).
template <int KH>
__global__ __launch_bounds__(64 * kRouteWaves) void small_route_kernel(const float* __restrict__ x,
                                                                       DeviceLayer L, Scratch S,
                                                                       int T, int n_route) {
  __shared__ __align__(16) float xl[kRouterTok][KH];
  __shared__ __align__(16) MfmaUnitSmem su;
  __shared__ int last;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int id = (int)blockIdx.x;
  if (id >= n_route) {
    if constexpr (KH <= 1280) {
      if (wave >= kMfmaWaves)
        __syncthreads();  // the unit's one barrier
      else if (L.quant_mode == kQuantNone)
        shared_gateup_mfma<kBF16, KH>(L, S, su, id - n_route, 0, T, T, true);
      else
        shared_gateup_mfma<kInt8, KH>(L, S, su, id - n_route, 0, T, T, true);
    }
    return;
  }
  const int bx = (L.E + 7) / 8, col = id % bx, pair = id / bx;
  // Waves 0 and 1: tokens 2p and 2p + 1 (one token per wave keeps the
  // router rows and the token row within the 128 VGPRs of a 16-wave
  // workgroup).
  const int t = kRouterTok * pair + wave;
  if (wave < kRouterTok && t < T) {
    const int ra = 8 * col + (lane >> 4), rb = ra + 4;
    RowPair<kBF16, KH> P;
    issue_rows(P, L.router, nullptr, L.E, L.H, ra, rb);
    RowStage<KH> X;
    load_row(X, x + (size_t)t * L.H, L.H, lane);
    store_row(X, xl[wave], L.H, lane);  // read back by this wave only
    float v0, v1;
    dot_rows(P, L.H, xl[wave], nullptr, nullptr, v0, v1);
    if ((lane & 15) == 0) {
      float* row = S.logits + (size_t)t * L.E;
      if (ra < L.E) __hip_atomic_store(row + ra, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (rb < L.E) __hip_atomic_store(row + rb, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's logit stores are complete
  __syncthreads();
  if (wave == 0) {
    if (lane == 0) {
      const int n = n_route;
      const int i = id % 8;
      int* sub = S.sync + kSmallRouteWord + 16 * i;
      int* top = S.sync + kSmallRouteWord + 16 * 8;
      int done = 0;
      if (__hip_atomic_fetch_add(sub, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
          (n - 1 - i) / 8) {
        __hip_atomic_store(sub, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int n_sub = n < 8 ? n : 8;
        if (__hip_atomic_fetch_add(top, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            n_sub - 1) {
          __hip_atomic_store(top, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          done = 1;
        }
      }
      last = done;
    }
  }
  __syncthreads();
  if (!last) return;
  route_dispatch(L, S, T, wave, lane);
}

// Routed tiles a dispatch can list: one per active group when every group
// fits one tile, else the dispatch's own bound.
int routed_bound(const DeviceLayer& L, int T, int tiles_bound, int mchunk) {
  return T <= mchunk ? min(L.E, T * L.K) : tiles_bound;
}

// Workgroups of a single-row pass: kSinglesGrid, or fewer where the groups
// that can hold one row (min(E, T k)) have fewer units.
dim3 singles_grid(const DeviceLayer& L, int T, int ur) {
  return dim3((unsigned)std::min<long long>(
      kSinglesGrid, std::min<long long>(L.E, (long long)T * L.K) * ur));
}

template <int KIND>
void launch_gateup_kind(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound,
                        int mchunk, hipStream_t s, bool shared_only) {
  if (mfma_shared(L, T)) {
    const bool in_router = shared_in_router(L, T);
    const int nsh = (T + kMfmaSharedRows - 1) / kMfmaSharedRows;
    const int sdn = in_router ? L.H / 16 : 0;
    const int sgu = in_router ? 0 : nsh * ((L.S + 15) / 16);
    const int units = sdn + sgu +
                      (shared_only ? 0 : routed_bound(L, T, tiles_bound, mchunk) * ((L.I + 15) / 16));
    const dim3 grid(units), block(256);
    if constexpr (KIND == kBF16) {
      batch_gateup_ms_kernel<kBF16, 1280, false><<<grid, block, 0, s>>>(L, S, T, mchunk, sdn, sgu);
    } else if (L.quant_mode == kQuantDynamic) {
      batch_gateup_ms_kernel<kInt8, 1280, true><<<grid, block, 0, s>>>(L, S, T, mchunk, sdn, sgu);
    } else {
      if (L.H <= 1280)
        batch_gateup_ms_kernel<kInt8, 1280, false><<<grid, block, 0, s>>>(L, S, T, mchunk, sdn, sgu);
      else
        batch_gateup_ms_kernel<kInt8, kWideK, false><<<grid, block, 0, s>>>(L, S, T, mchunk, sdn, sgu);
    }
    return;
  }
  const int nsh = (T + kSharedRows - 1) / kSharedRows;
  const int units = nsh * ((L.S + 15) / 16) +
                    (shared_only ? 0 : routed_bound(L, T, tiles_bound, mchunk) * ((L.I + 15) / 16));
  const dim3 grid(units), block(256);
  if (L.quant_mode == kQuantDynamic) {
    if (L.H <= 1280)
      batch_gateup_kernel<KIND, 1280, true><<<grid, block, 0, s>>>(L, S, T, mchunk, nsh);
    else
      batch_gateup_kernel<KIND, kWideK, true><<<grid, block, 0, s>>>(L, S, T, mchunk, nsh);
  } else {
    if (L.H <= 1280)
      batch_gateup_kernel<KIND, 1280, false><<<grid, block, 0, s>>>(L, S, T, mchunk, nsh);
    else
      batch_gateup_kernel<KIND, kWideK, false><<<grid, block, 0, s>>>(L, S, T, mchunk, nsh);
  }
}

}  // namespace

bool batch_supported(const DeviceLayer& L) {
  // Down rows are held as one segment up to kSegK or as two halves.
  return L.H <= kWideK && L.S <= kWideK && L.I <= kWideK && L.I % 16 == 0 && L.S % 16 == 0 &&
         L.H % 32 == 0;
}

void launch_batch_gateup(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound,
                         int mchunk, hipStream_t s, bool shared_only) {
  if (L.quant_mode == 0)
    launch_gateup_kind<kBF16>(L, S, T, tiles_bound, mchunk, s, shared_only);
  else
    launch_gateup_kind<kInt8>(L, S, T, tiles_bound, mchunk, s, shared_only);
}

void launch_singles_gateup(const DeviceLayer& L, const Scratch& S, int T, hipStream_t s) {
  const dim3 grid = singles_grid(L, T, (L.I + 15) / 16), block(256);
  if (L.H <= 1280)
    singles_gateup_kernel<1280><<<grid, block, 0, s>>>(L, S);
  else
    singles_gateup_kernel<kWideK><<<grid, block, 0, s>>>(L, S);
}

void launch_singles_down(const DeviceLayer& L, const Scratch& S, int T, hipStream_t s) {
  const dim3 grid = singles_grid(L, T, down_units(L.H, L.I)), block(256);
  if (L.I <= kSegK)
    singles_down_kernel<false><<<grid, block, 0, s>>>(L, S);
  else
    singles_down_kernel<true><<<grid, block, 0, s>>>(L, S);
}

void launch_batch_down(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound, int mchunk,
                       hipStream_t s, bool shared_only) {
  const int nsh = (T + kSharedRows - 1) / kSharedRows;
  const int units = nsh * down_units(L.H, L.S) +
                    (shared_only ? 0 : routed_bound(L, T, tiles_bound, mchunk) * down_units(L.H, L.I));
  const dim3 grid(units), block(256);
  if (mfma_shared(L, T)) {
    const int sdn = shared_in_router(L, T) ? 0
                                           : (T + kMfmaSharedRows - 1) / kMfmaSharedRows * (L.H / 32);
    const dim3 grid16(sdn + (shared_only ? 0 : routed_bound(L, T, tiles_bound, mchunk) *
                                                   down_units(L.H, L.I)));
    if (L.quant_mode == kQuantNone)
      batch_down_ms_kernel<kBF16, false><<<grid16, block, 0, s>>>(L, S, T, mchunk, sdn);
    else if (L.quant_mode == kQuantDynamic)
      batch_down_ms_kernel<kInt8, true><<<grid16, block, 0, s>>>(L, S, T, mchunk, sdn);
    else
      batch_down_ms_kernel<kInt8, false><<<grid16, block, 0, s>>>(L, S, T, mchunk, sdn);
    return;
  }
  if (L.quant_mode == 0)
    batch_down_kernel<kBF16, false><<<grid, block, 0, s>>>(L, S, T, mchunk, nsh);
  else if (L.quant_mode == kQuantDynamic)
    batch_down_kernel<kInt8, true><<<grid, block, 0, s>>>(L, S, T, mchunk, nsh);
  else
    batch_down_kernel<kInt8, false><<<grid, block, 0, s>>>(L, S, T, mchunk, nsh);
}

void launch_small_route(const float* x, const DeviceLayer& L, const Scratch& S, int T,
                        hipStream_t s) {
  const int n_route = (L.E + 7) / 8 * ((T + kRouterTok - 1) / kRouterTok);
  const int sgu = shared_in_router(L, T) ? (L.S + 15) / 16 : 0;
  const dim3 grid(n_route + sgu);
  if (L.H <= 1280)
    small_route_kernel<1280><<<grid, dim3(64 * kRouteWaves), 0, s>>>(x, L, S, T, n_route);
  else
    small_route_kernel<kWideK><<<grid, dim3(64 * kRouteWaves), 0, s>>>(x, L, S, T, n_route);
}

}  // namespace uocr
