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

namespace uocr {

namespace {

enum { kBF16 = 0, kInt8 = 1, kW8A8 = 2 };
constexpr int kLpr = 16;        // lanes per weight row
constexpr int kWide = 2048;     // widest reduction dimension (H, S)
constexpr int kNarrow = 1024;   // widest routed intermediate size (I)
constexpr int kMaxK = 8;        // most routed experts per token
// Offset marker past every buffer (buffers are < 1 GiB, so a sum of two
// markers stays out of range too).
constexpr uint32_t kOut = 0x40000000u;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // Raw buffer: stride 0, range-checked against `bytes` (gfx9 word 3).
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Quantise an FP32 row held in LDS per 32-block (Int8Matrix::quantize,
// src/cpu/quantized.rs:43-74) with the 64 lanes of one wave; non-finite
// input or an underflowing scale raises Numerical.
__device__ void quantize_lds(const float* xl, int K, int8_t* xq, float* xs, int lane, int* err) {
  for (int b = lane; b < K / kQBlock; b += 64) {
    const float* v = xl + b * kQBlock;
    float maximum = 0.0f;
    bool bad = false;
    for (int i = 0; i < kQBlock; i++) {
      bad |= !isfinite(v[i]);
      maximum = fmaxf(maximum, fabsf(v[i]));
    }
    const float scale = maximum / 127.0f;
    if (bad || (maximum > 0.0f && scale == 0.0f)) raise_error(err, kErrNumerical);
    xs[b] = scale;
    for (int i = 0; i < kQBlock; i++) {
      int q = 0;
      if (scale != 0.0f) q = (int)fminf(fmaxf(rintf(v[i] / scale), -127.0f), 127.0f);
      xq[b * kQBlock + i] = (int8_t)q;
    }
  }
}

// 16-byte weight chunks of two rows, ra and rb, of a row-major [rows, K]
// matrix with K <= KMAX: the lane takes chunks j, j + 16, ... of both rows
// (j = lane % 16), so the four 16-lane groups of a wave cover 8 rows.
template <int KIND, int KMAX>
struct RowPair {
  static constexpr int kElems = KIND == kBF16 ? 8 : 16;   // elements per chunk
  static constexpr int kC = KMAX / kElems / kLpr;          // chunks per lane per row
  u32x4 wa[kC], wb[kC];
  float sa[kC], sb[kC];
};

// Issues every load of a RowPair. Rows outside [0, rows) and chunks past K
// read as zero; `w` / `s` are the matrix and (INT8) its [rows, K/32] scales.
template <int KIND, int KMAX>
__device__ __forceinline__ void issue_rows(RowPair<KIND, KMAX>& P, const void* w, const float* s,
                                           int rows, int K, int ra, int rb) {
  using RP = RowPair<KIND, KMAX>;
  constexpr int kBytes = KIND == kBF16 ? 2 : 1;
  const int j = threadIdx.x & (kLpr - 1);
  const int nchunks = K / RP::kElems;
  const uint32_t row_bytes = (uint32_t)K * kBytes;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, (uint32_t)rows * row_bytes);
  const uint32_t oa = ra >= 0 && ra < rows ? (uint32_t)ra * row_bytes : kOut;
  const uint32_t ob = rb >= 0 && rb < rows ? (uint32_t)rb * row_bytes : kOut;
  if constexpr (KIND == kBF16) {
#pragma unroll
    for (int m = 0; m < RP::kC; m++) {
      const int c = j + kLpr * m;
      const uint32_t co = c < nchunks ? (uint32_t)c * 16u : kOut;
      P.wa[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, oa + co, 0, 0);
      P.wb[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, ob + co, 0, 0);
    }
  } else {
    // Each chunk's scales are issued with its weights, so chunk m can be
    // used as soon as its four loads are back.
    const int nblk = K / kQBlock;
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(s, (uint32_t)rows * nblk * 4u);
    const uint32_t sa = ra >= 0 && ra < rows ? (uint32_t)ra * nblk * 4u : kOut;
    const uint32_t sb = rb >= 0 && rb < rows ? (uint32_t)rb * nblk * 4u : kOut;
#pragma unroll
    for (int m = 0; m < RP::kC; m++) {
      const int c = j + kLpr * m;
      const uint32_t co = c < nchunks ? (uint32_t)c * 16u : kOut;
      const uint32_t bo = c < nchunks ? (uint32_t)(c >> 1) * 4u : kOut;
      P.wa[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, oa + co, 0, 0);
      P.wb[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, ob + co, 0, 0);
      P.sa[m] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(sr, sa + bo, 0, 0));
      P.sb[m] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(sr, sb + bo, 0, 0));
    }
  }
}

// Dots both rows with the LDS activation row (xl, or xq/xs for W8A8);
// every lane of a 16-lane group returns that group's two row sums.
template <int KIND, int KMAX>
__device__ __forceinline__ void dot_rows(const RowPair<KIND, KMAX>& P, int K, const float* xl,
                                         const int8_t* xq, const float* xs, float& r0,
                                         float& r1) {
  using RP = RowPair<KIND, KMAX>;
  const int j = threadIdx.x & (kLpr - 1);
  const int nchunks = K / RP::kElems;
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int m = 0; m < RP::kC; m++) {
    const int c = j + kLpr * m;
    if (c >= nchunks) break;
    const u32x4 va = P.wa[m], vb = P.wb[m];
    if constexpr (KIND == kBF16) {
      const float4* xp = reinterpret_cast<const float4*>(xl + c * 8);
      const float4 x0 = xp[0], x1 = xp[1];
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        a0 = fmaf(bf16_lo(va[i]), xv[2 * i], a0);
        a0 = fmaf(bf16_hi(va[i]), xv[2 * i + 1], a0);
        a1 = fmaf(bf16_lo(vb[i]), xv[2 * i], a1);
        a1 = fmaf(bf16_hi(vb[i]), xv[2 * i + 1], a1);
      }
    } else if constexpr (KIND == kInt8) {
      const float4* xp = reinterpret_cast<const float4*>(xl + c * 16);
#pragma unroll
      for (int v4 = 0; v4 < 4; v4++) {
        const float4 xv = xp[v4];
        const float x4[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int b = 0; b < 4; b++) {
          // The reference multiplies the dequantised (rounded) weight by x.
          const float da = (float)(int8_t)((va[v4] >> (8 * b)) & 0xff) * P.sa[m];
          const float db = (float)(int8_t)((vb[v4] >> (8 * b)) & 0xff) * P.sb[m];
          a0 = fmaf(da, x4[b], a0);
          a1 = fmaf(db, x4[b], a1);
        }
      }
    } else {
      const int4 xv = *reinterpret_cast<const int4*>(xq + c * 16);
      int pa = __builtin_amdgcn_sdot4((int)va.x, xv.x, 0, false);
      pa = __builtin_amdgcn_sdot4((int)va.y, xv.y, pa, false);
      pa = __builtin_amdgcn_sdot4((int)va.z, xv.z, pa, false);
      pa = __builtin_amdgcn_sdot4((int)va.w, xv.w, pa, false);
      int pb = __builtin_amdgcn_sdot4((int)vb.x, xv.x, 0, false);
      pb = __builtin_amdgcn_sdot4((int)vb.y, xv.y, pb, false);
      pb = __builtin_amdgcn_sdot4((int)vb.z, xv.z, pb, false);
      pb = __builtin_amdgcn_sdot4((int)vb.w, xv.w, pb, false);
      // Chunks 2b and 2b+1 (lanes j, j^1) form block b: exact i32 sum.
      const int ia = pa + __shfl_xor(pa, 1);
      const int ib = pb + __shfl_xor(pb, 1);
      if ((j & 1) == 0) {
        const int b = c >> 1;
        a0 += (float)ia * P.sa[m] * xs[b];
        a1 += (float)ib * P.sb[m] * xs[b];
      }
    }
  }
  r0 = row16_sum(a0);
  r1 = row16_sum(a1);
}

// An FP32 row of n <= N values (n % 4 == 0) held in registers of one wave
// (float4 at lane, lane + 64, ...): load_row issues every load, store_row
// writes the row into LDS.
template <int N>
struct RowStage {
  static constexpr int kV = N / 4 / 64;
  u32x4 v[kV];
};
template <int N>
__device__ __forceinline__ void load_row(RowStage<N>& R, const float* src, int n, int lane) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(src, (uint32_t)n * 4u);
#pragma unroll
  for (int i = 0; i < RowStage<N>::kV; i++) {
    const int at = lane + 64 * i;
    R.v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, at * 4 < n ? (uint32_t)at * 16u : kOut, 0, 0);
  }
}
template <int N>
__device__ __forceinline__ void store_row(const RowStage<N>& R, float* dst, int n, int lane) {
#pragma unroll
  for (int i = 0; i < RowStage<N>::kV; i++) {
    const int at = lane + 64 * i;
    if (at * 4 < n) reinterpret_cast<u32x4*>(dst)[at] = R.v[i];
  }
}

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
