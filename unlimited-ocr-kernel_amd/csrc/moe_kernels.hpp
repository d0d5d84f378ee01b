// Internal interface between the C-ABI layer (api.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace uocr {

// Expert "groups": 0..E-1 are the routed experts, E is the fused shared
// expert (width S = I * n_shared_experts).
// uocr_quant_mode values (uocr_moe.h), for device code.
constexpr int kQuantNone = 0, kQuantWeightsOnly = 1, kQuantDynamic = 2;

struct DeviceLayer {
  int H, I, S, E, K;
  int normalize;
  float scale;
  float eps;
  int quant_mode;            // uocr_quant_mode
  const uint16_t* router;    // [E,H] bf16
  // BF16 expert weights. w13 holds per group [2W,H]: gate and up rows
  // interleaved in blocks of 32 (gate j..j+31, then up j..j+31, ...).
  // w2 holds per group the down matrix [H,W] unchanged.
  const uint16_t* w13;
  const uint16_t* w2;
  // INT8 overlay with the same row order; scales [rows, cols/32].
  const int8_t* q13;
  const float* s13;
  const int8_t* q2;
  const float* s2;
  const float* norm_w;       // [H] post-attention RMSNorm weight (f32)
  // The MFMA engine's copies of w13 / w2 (BF16) and q13 / q2 (INT8 overlay)
  // in k-blocked panels: each group's [N rows, K] matrix as [K/32][N][32],
  // so the 32-deep stage of a row tile is one contiguous run (same group
  // offsets as the row-major arrays).
  const uint16_t* w13k;
  const uint16_t* w2k;
  const int8_t* q13k;
  const int8_t* q2k;
  // The one-token engine's copy of s2 block-major: each group's [H, W/32]
  // scales as [W/32][H] (same group offsets), so one 32-block's scales of
  // every output feature are one contiguous run.
  const float* s2k;
  // The MFMA engines' copy of s13 block-major ([H/32][2W] per group, same
  // group offsets).
  const float* s13k;

  __host__ __device__ int width(int g) const { return g < E ? I : S; }
  __host__ __device__ size_t n13() const { return ((size_t)E * 2 * I + 2 * (size_t)S) * H; }
  __host__ __device__ size_t n2() const { return ((size_t)E * I + S) * H; }
  __host__ __device__ size_t w13_offset(int g) const { return (size_t)g * 2 * I * H; }
  __host__ __device__ size_t w2_offset(int g) const { return (size_t)g * H * I; }
  __host__ __device__ size_t s13_offset(int g) const { return (size_t)g * 2 * I * (H / 32); }
  __host__ __device__ size_t s2_offset(int g) const { return (size_t)g * H * (I / 32); }
};

// Optional trace of the W8A8 (DynamicActivations, single-row group)
// projections: exact i32 block sums in checkpoint row order and the f32
// hidden rows that entered the down projection. Routed entries are indexed
// by dispatched position p: gate/up [p][2I][H/32] (gate rows, then up
// rows), down [p][H][I/32], hidden [p][I]. Shared entries exist for one
// token only: gate/up [2S][H/32], down [H][S/32], hidden [S]. Null
// pointers are not written.
struct Q8Trace {
  int32_t* gateup = nullptr;
  int32_t* down = nullptr;
  float* hidden = nullptr;
  int32_t* s_gateup = nullptr;
  int32_t* s_down = nullptr;
  float* s_hidden = nullptr;
};

// Per-forward device scratch carved from the context's reservation.
// Stamps per workgroup row of the decode engine's timeline.
constexpr int kDecodeStamps = 8;

struct Scratch {
  float* logits;    // [T,E]
  int* topk_ids;    // [T,K]
  float* topk_w;    // [T,K]
  int* offsets;     // [E+1] expert start in the dispatched order
  int* perm_rows;   // [T*K] token of each assignment
  float* perm_w;    // [T*K]
  int* inv_pos;     // [T*K] position of (token, slot) in the dispatched order
  int* tiles;       // [max_tiles*2] (group, first row) per row tile
  int* counters;    // [4]: row tiles, routed row tiles
  int* chunk_counts;  // [ceil(T/16), 64] per-chunk expert counts (router)
  // Small router (T <= 16): one record of kTileDescInts per routed tile
  // (group, first dispatched position, rows, one unused word, then the
  // rows' tokens), so that a unit reads its tile with one load; null: none
  // (units read the tile list, the expert offsets and the permutation).
  int* tile_desc;
  float* h;         // [T*K, I] routed hidden in dispatched order
  float* hs;        // [T, S] shared hidden
  float* y;         // [T*K, H] routed expert outputs in dispatched order
  float* ys;        // [T, H] shared expert output
  float* xn;        // [T, H] normalised block input
  uint16_t* xb;     // [2][H/32][T][32] bf16 planes (hi, lo) of the layer input (MFMA engine)
  float* gu;        // one token: hidden rows, routed [K, I] (ascending slot) then shared [S]
  int8_t* q8x;      // int8 mode: quantised input [T, H] and hidden rows [T*K*I + T*S]
  float* router_part;  // router_part_bytes(T, H): the split router's partial logits
  float* q8s;       // int8 mode: their block scales [T*H/32 + (T*K*I + T*S)/32]
  int* err;         // device error flag
  int* sync;        // kDecodeSyncBytes: the decode engine's counts and flags (zero between launches)
  float* part;      // kDecodePartBytes: the decode engine's down partials (0xffffffff between launches)
  int wait_limit;   // the decode engine's wait bound in polls (< 0: its default)
  Q8Trace q8;       // W8A8 trace (tests), all null by default
  // The decode engine's timeline: kDecodeStamps real-time stamps per
  // workgroup of its launch (uocr_moe_trace::decode_stamps), null: none.
  unsigned long long* stamps = nullptr;
};

int max_tiles(int T, int K, int E, int bm);
constexpr int kTileDescInts = 32;  // one 128-byte line per record

// route.hip
void launch_router_logits(const float* x, const uint16_t* w, int T, int H, int E, float* logits,
                          hipStream_t s);
void launch_topk(const float* logits, int T, int E, int K, int normalize, float scale, int* ids,
                 float* weights, int* err, hipStream_t s);

// The fused router covers hidden widths up to 2048 (64 K steps of 32).
inline bool router_mfma_supported(int H) { return H % 32 == 0 && H <= 2048; }
// x_hi (and x_lo) set: also writes the bf16 hi (and lo) planes of x that
// the MFMA grouped GEMM reads ([H/32][T][32]), as launch_split_planes would.
// part and route_counts set: few tokens split H over router_ksplit(T, H)
// workgroups per 16-token chunk (partial logits in part, router_part_bytes
// of them); the chunk's last workgroup adds them in order and routes.
// route_counts: one word per chunk (stride 16), zero before the launch and
// zero again after it.
void launch_router_topk_mfma(const float* x, const uint16_t* w, int T, int H, int E, int K,
                             int normalize, float scale, float* logits, int* ids, float* weights,
                             int* chunk_counts, uint16_t* x_hi, uint16_t* x_lo, int* err,
                             float* part, int* route_counts, hipStream_t s);
// Workgroups per 16-token chunk of the router: enough for ~256 workgroups
// in all, at most 8 and at most one 32-wide step of H per workgroup's wave.
inline int router_ksplit(int T, int H) {
  const int chunks = (T + 15) / 16, steps = H / 32;
  int k = 256 / (chunks > 0 ? chunks : 1);
  k = k > 8 ? 8 : k;
  k = k > steps ? steps : k;
  return k < 2 ? 1 : k;
}
inline size_t router_part_bytes(int T, int H) {
  const int k = router_ksplit(T, H);
  return k > 1 ? (size_t)((T + 15) / 16) * k * 16 * 64 * 4 : 0;
}

// dispatch.hip
// narrow > 0 moves each expert's last tile of at most `narrow` rows into a
// second routed list (counters[2] = tiles of the first list).
void launch_dispatch_chunked(const int* ids, const float* w, int T, int E, int K, int bm,
                             int narrow, const int* chunk_counts, int* offsets, int* perm_rows, float* perm_w,
                             int* inv_pos, int* tiles, int* counters, hipStream_t s);
void launch_dispatch(const int* ids, const float* w, int T, int E, int K, int bm, int narrow,
                     int* offsets,
                     int* perm_rows, float* perm_w, int* inv_pos, int* tiles, int* counters,
                     hipStream_t s);

// batch.hip: small-batch expert engine over row tiles of <= 16 tokens (FP32
// math, INT8 weight-only and W8A8), and the small-batch router (T <= 16):
// logits, then one workgroup that routes and builds the dispatch.
bool batch_supported(const DeviceLayer& L);
// shared_only: the shared expert's units only (the MFMA engine at one
// token under DynamicActivations, where the shared group is a single row).
void launch_batch_gateup(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound,
                         int mchunk, hipStream_t s, bool shared_only = false);
void launch_batch_down(const DeviceLayer& L, const Scratch& S, int T, int tiles_bound, int mchunk,
                       hipStream_t s, bool shared_only = false);
// The routed groups of exactly one row of an INT8 DynamicActivations layer
// (W8A8 row by row) beside the MFMA engine, after its dispatch.
void launch_singles_gateup(const DeviceLayer& L, const Scratch& S, int T, hipStream_t s);
void launch_singles_down(const DeviceLayer& L, const Scratch& S, int T, hipStream_t s);
// Router logits, routing and dispatch of T <= 16 tokens in one launch
// (its workgroups counted in the words from kSmallRouteWord of S.sync,
// which are zero between launches).
void launch_small_route(const float* x, const DeviceLayer& L, const Scratch& S, int T,
                        hipStream_t s);

// gemv.hip: single-matrix operator kernels.
// Operator entry points (single matrix).
void launch_linear_bf16(const float* x, int m, int k, const uint16_t* w, int n, float* y,
                        hipStream_t s);
void launch_int8_linear(const int8_t* q, const float* sc, int rows, int cols, const float* x,
                        int batch, float* y, hipStream_t s);
void launch_int8_dynamic(const int8_t* q, const float* sc, int rows, int cols, const float* x,
                         float* y, int32_t* block_sums, int8_t* xq, float* xs, int* err,
                         hipStream_t s);
void gemv_init_attributes();

// gemm.hip: MFMA grouped GEMM engine. Activations enter as bf16 planes
// (hi, and lo for FP32-class precision).
struct MfmaPlanes {
  uint16_t* x_hi;   // [H/32][T][32] (k-blocked)
  uint16_t* x_lo;
  uint16_t* h_hi;   // [T*K, I] routed hidden, dispatched order
  uint16_t* h_lo;
  uint16_t* hs_hi;  // [T, S] shared hidden
  uint16_t* hs_lo;
};
void launch_split_planes(const float* x, int rows, int K, uint16_t* hi, uint16_t* lo,
                         hipStream_t s);
// lists: kListShared, kListRouted or both (the items each launch runs).
constexpr int kListShared = 1, kListRouted = 2, kListAll = 3;
void launch_mfma_gateup(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, int lists, hipStream_t s);
void launch_mfma_down(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                      int tiles_bound, bool bf16_only, int lists, hipStream_t s);
constexpr int kMfmaBM = 256;
constexpr int kMfmaQ8BM = 64;  // INT8 weights: 64-row tiles, 64 x 512 items
void mfma_init_attributes();
// out = `groups` row-major [N, K] matrices (elem_bytes 1 or 2, K % 32 == 0,
// matrix g at g * N * K) as k-blocked panels [K/32][N][32].
// out = in transposed per matrix: `groups` row-major f32 [rows, cols]
// matrices to [cols, rows] (the block-major down scales).
void launch_transpose_f32(const float* in, float* out, int rows, int cols, int groups,
                          hipStream_t s);
void launch_panelize(const void* in, void* out, int elem_bytes, int N, int K, int groups,
                     hipStream_t s);

// gemm_i8.hip: int8 x int8 grouped GEMM with int32 block accumulation (the
// opt-in UOCR_FLAG_INT8_MFMA mode). Activations enter quantised per 32-block.
struct I8Planes {
  const int8_t* xq;     // [T, H] quantised layer input
  const float* xs;      // [T, H/32] its block scales
  float* hid;           // [T*K, I] routed hidden rows (dispatched order), FP32
  float* hid_shared;    // [T, S] shared-expert hidden rows, FP32
  int8_t* hid_q;        // the hidden rows quantised: [T*K, I] then [T, S]
  float* hid_s;         // their block scales: [T*K, I/32] then [T, S/32]
};
constexpr int kI8BM = 64;  // token rows per row tile
bool i8_supported(const DeviceLayer& L);
bool i8_traced(const Scratch& S, int T);  // traced GEMMs: FP32 hidden rows + quantize_rows_kernel
void launch_quantize_rows(const float* src, int rows, int K, int8_t* dst, float* sc,
                          const float* src2, int rows2, int K2, int8_t* dst2, float* sc2,
                          int* err, hipStream_t s);
void launch_i8_gateup(const DeviceLayer& L, const Scratch& S, const I8Planes& P, int T,
                      int tiles_bound, hipStream_t s);
void launch_i8_down(const DeviceLayer& L, const Scratch& S, const I8Planes& P, int T,
                    int tiles_bound, hipStream_t s);
constexpr int kGemvChunk = 16;

// decode.hip: one-token expert engine, one launch (router logits, the
// shared and the routed gate/up with their shares of the down projection,
// ordered combine into out), ordered inside by the kDecodeSyncBytes at
// S.sync, which must be zero when it starts and are zero again when it
// ends, and handing its logits and down partials over through the
// kDecodePartBytes at S.part, which must hold 0xffffffff in every byte
// when it starts and do again when it ends.
constexpr size_t kDecodeSyncBytes = 64 << 10;
// Partials: (S/32 + K I/32) per output feature, at most (2048/32 + 8 *
// 1024/32) x 2048 features, 4 bytes each; then a 64-word copy of the
// router logits per routed gate/up workgroup (at most 8 * 1024/32 = 256).
constexpr size_t kDecodePartBytes = (size_t)(2048 / 32 + 8 * 1024 / 32 + 8) * 2048 * 4;
// The split router's per-chunk counts (<= 128 chunks, one word per 64 bytes)
// live in the same zero-between-launches region, past the decode engine's
// words (at most 1 + 16 + 2 * 256 lines).
constexpr size_t kRouterSyncWord = 10240;
static_assert((kRouterSyncWord + 128 * 16) * 4 <= kDecodeSyncBytes, "router counts fit");
static_assert((1 + 16 + 2 * 256) * 16 <= kRouterSyncWord, "after the decode words");
// The small-batch router's counts of logit workgroups done (8 sub-count
// lines and a top line, past the split router's counts).
constexpr size_t kSmallRouteWord = kRouterSyncWord + 128 * 16;
static_assert((kSmallRouteWord + 9 * 16) * 4 <= kDecodeSyncBytes, "small router counts fit");
// By the layer's kind: BF16 layers take the row-dot engine (decode_rows.hip:
// down rows on workgroups of their own, hidden values handed over through
// the sync words), INT8 overlays the split-K engine (decode.hip).
bool decode_supported(const DeviceLayer& L);
void launch_decode(const DeviceLayer& L, const Scratch& S, const float* residual, float* out,
                   hipStream_t s);
bool rows_decode_supported(const DeviceLayer& L);
void launch_rows_decode(const DeviceLayer& L, const Scratch& S, const float* residual, float* out,
                        hipStream_t s);

// combine.hip
// RMSNorm output of rows: the normalised rows (out, [T, H]) and optionally
// their bf16 planes (hi, and lo for FP32-class precision), k-blocked
// ([H/32][T][32]) as the MFMA engine reads them.
struct RowNorm {
  const float* w = nullptr;
  float eps = 0.0f;
  float* out = nullptr;
  uint16_t* hi = nullptr;
  uint16_t* lo = nullptr;
};
// Combine; with `next`, also the following layer's RMSNorm of the result.
// y16: the expert outputs are bf16 rows (MFMA engine, BF16 activations).
void launch_combine(const Scratch& S, const float* residual, int T, int H, int K, float* out,
                    const RowNorm* next, bool y16, hipStream_t s);
// Rows of width <= 2048 (multiple of 4) take the fused norm (planes too);
// wider rows a plain one (no planes).
bool row_norm_fusable(int width);
bool row_norm_wave(int width);
void launch_rms_norm(const float* x, int rows, int width, const RowNorm& nn, int* err,
                     hipStream_t s);

// lmhead.hip: the vocabulary projection of one hidden row.
struct LmHeadView {
  int V = 0, H = 0;
  int kind = 0;                 // 0 BF16, 1 INT8 weight-only, 2 W8A8
  float eps = 0.0f;
  const float* norm_w = nullptr;  // [H] f32
  const uint16_t* w = nullptr;    // [V, H] bf16
  const int8_t* q = nullptr;      // [V, H]
  const float* s = nullptr;       // [V, H/32]
};
// The one-launch path: widths that are multiples of 64, up to 2048.
bool lm_head_fast(int H);
// logits[V] of `hidden` (one row of H): RMSNorm, then the projection.
void launch_lm_head(const float* hidden, const LmHeadView& head, float* logits, int* err,
                    hipStream_t s);

}  // namespace uocr
