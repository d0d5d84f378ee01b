// Row-dot building blocks shared by the small-batch expert engines: two
// weight rows per lane (16 lanes per row, 8 rows per wave), every 16-byte
// chunk loaded with a range-checked buffer load before any is used.
//
// Arithmetic is that of Decoder::projection (src/decoder/mod.rs:99-112):
// BF16 weights widened exactly; INT8 weight-only as q * x summed over each
// 16-byte chunk and scaled once by its block scale (the reference rounds
// w = q * scale first, src/cpu/quantized.rs:119-131); W8A8 with the
// activation row quantised per 32-block and exact i32 block sums
// (src/cpu/quantized.rs:155-236). Only the FP32 summation order (and, for
// INT8, where the scale is applied) differs.
#pragma once

#include "common.hpp"

namespace uocr {

enum { kBF16 = 0, kInt8 = 1, kW8A8 = 2 };
constexpr int kLpr = 16;  // lanes per weight row
// Offset marker past every buffer (buffers are < 1 GiB, so a sum of two
// markers stays out of range too).
constexpr uint32_t kOut = 0x40000000u;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // Raw buffer: stride 0, range-checked against `bytes` (gfx9 word 3).
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Quantise an FP32 row held in LDS per 32-block (Int8Matrix::quantize,
// src/cpu/quantized.rs:43-74) with waves `wave` of `nw`: a wave takes two
// blocks per step, one value per lane, and four steps at once (independent
// chains, so their latencies overlap); the block maximum comes from lane
// moves (the maximum of absolute values is the same in any order, so the
// scale and the rounded values are those of the serial loop). Non-finite
// input or an underflowing scale raises Numerical. Every lane of each
// calling wave must call it.
__device__ inline void quantize_lds_waves(const float* xl, int K, int8_t* xq, float* xs, int wave,
                                          int nw, int lane, int* err) {
  constexpr int kU = 4;
  const int nb = K / kQBlock;
  const int half = lane >> 5, i = lane & 31;
  const int step = 2 * nw;
  for (int b0 = 2 * wave; b0 < nb; b0 += step * kU) {
    float v[kU], m[kU];
    unsigned long long nonfinite[kU];
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int b = b0 + step * u + half;
      v[u] = b < nb ? xl[b * kQBlock + i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kU; u++) {
      nonfinite[u] = __ballot(!isfinite(v[u]));
      m[u] = half_wave_max(fabsf(v[u]));
    }
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int b = b0 + step * u + half;
      const float scale = m[u] / 127.0f;
      if (b < nb) {
        if (i == 0) {
          const bool bad = ((half ? nonfinite[u] >> 32 : nonfinite[u]) & 0xffffffffull) != 0;
          if (bad || (m[u] > 0.0f && scale == 0.0f)) raise_error(err, kErrNumerical);
          xs[b] = scale;
        }
        int q = 0;
        if (scale != 0.0f) q = (int)fminf(fmaxf(rintf(v[u] / scale), -127.0f), 127.0f);
        xq[b * kQBlock + i] = (int8_t)q;
      }
    }
  }
}
// The same with one wave.
__device__ inline void quantize_lds(const float* xl, int K, int8_t* xq, float* xs, int lane, int* err) {
  quantize_lds_waves(xl, K, xq, xs, 0, 1, lane, err);
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

// Issues every load of a RowPair: two row segments of a row-major
// [rows, ld] matrix, columns [ca, ca + K) of row ra and [cb, cb + K) of row
// rb (ca, cb multiples of 32). Rows outside [0, rows) and chunks past the
// segment or the row read as zero; `w` / `s` are the matrix and (INT8) its
// [rows, ld/32] scales.
template <int KIND, int KMAX>
__device__ __forceinline__ void issue_segs(RowPair<KIND, KMAX>& P, const void* w, const float* s,
                                           int rows, int ld, int ra, int ca, int rb, int cb,
                                           int K) {
  using RP = RowPair<KIND, KMAX>;
  constexpr int kBytes = KIND == kBF16 ? 2 : 1;
  const int j = threadIdx.x & (kLpr - 1);
  const int na = min(K, ld - ca) / RP::kElems, nb = min(K, ld - cb) / RP::kElems;
  const uint32_t row_bytes = (uint32_t)ld * kBytes;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, (uint32_t)rows * row_bytes);
  const uint32_t oa = ra >= 0 && ra < rows ? (uint32_t)ra * row_bytes + (uint32_t)ca * kBytes : kOut;
  const uint32_t ob = rb >= 0 && rb < rows ? (uint32_t)rb * row_bytes + (uint32_t)cb * kBytes : kOut;
  if constexpr (KIND == kBF16) {
#pragma unroll
    for (int m = 0; m < RP::kC; m++) {
      const int c = j + kLpr * m;
      P.wa[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, oa + (c < na ? (uint32_t)c * 16u : kOut), 0, 0);
      P.wb[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, ob + (c < nb ? (uint32_t)c * 16u : kOut), 0, 0);
    }
  } else {
    // Each chunk's scales are issued with its weights, so chunk m can be
    // used as soon as its four loads are back.
    const int nblk = ld / kQBlock;
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(s, (uint32_t)rows * nblk * 4u);
    const uint32_t sa = ra >= 0 && ra < rows ? ((uint32_t)ra * nblk + (uint32_t)(ca / kQBlock)) * 4u : kOut;
    const uint32_t sb = rb >= 0 && rb < rows ? ((uint32_t)rb * nblk + (uint32_t)(cb / kQBlock)) * 4u : kOut;
#pragma unroll
    for (int m = 0; m < RP::kC; m++) {
      const int c = j + kLpr * m;
      P.wa[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, oa + (c < na ? (uint32_t)c * 16u : kOut), 0, 0);
      P.wb[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, ob + (c < nb ? (uint32_t)c * 16u : kOut), 0, 0);
      P.sa[m] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(sr, sa + (c < na ? (uint32_t)(c >> 1) * 4u : kOut), 0, 0));
      P.sb[m] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(sr, sb + (c < nb ? (uint32_t)(c >> 1) * 4u : kOut), 0, 0));
    }
  }
}

// Columns [c0, c0 + K) of rows ra and rb.
template <int KIND, int KMAX>
__device__ __forceinline__ void issue_rows_cols(RowPair<KIND, KMAX>& P, const void* w,
                                                const float* s, int rows, int ld, int c0, int K,
                                                int ra, int rb) {
  issue_segs(P, w, s, rows, ld, ra, c0, rb, c0, K);
}

// Rows ra and rb of a row-major [rows, K] matrix with K <= KMAX.
template <int KIND, int KMAX>
__device__ __forceinline__ void issue_rows(RowPair<KIND, KMAX>& P, const void* w, const float* s,
                                           int rows, int K, int ra, int rb) {
  issue_rows_cols(P, w, s, rows, K, 0, K, ra, rb);
}

// Where a W8A8 dot also stores its exact i32 block sums (a test trace):
// blocks [0, na) of segment a at a[...], [0, nb) of segment b at b[...];
// null pointers store nothing.
struct BlockSumOut {
  int32_t* a = nullptr;
  int32_t* b = nullptr;
  int na = 0, nb = 0;
};

// Dots both rows with the LDS activation row (xl, or xq/xs for a W8A8
// dot); every lane of a 16-lane group returns that group's two row sums.
// DOT picks the arithmetic: INT8 chunks serve both the weight-only and the
// W8A8 dot. The b segment reads the row from element xb_off on (a multiple
// of 32; 0 when both segments cover the same columns).
template <int DOT, int KIND, int KMAX>
__device__ __forceinline__ void dot_rows_as(const RowPair<KIND, KMAX>& P, int K, const float* xl,
                                            const int8_t* xq, const float* xs, float& r0,
                                            float& r1, int xb_off = 0,
                                            const BlockSumOut& sums = BlockSumOut()) {
  using RP = RowPair<KIND, KMAX>;
  static_assert((DOT == kBF16) == (KIND == kBF16), "BF16 dots need BF16 chunks");
  const int j = threadIdx.x & (kLpr - 1);
  const int nchunks = K / RP::kElems;
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int m = 0; m < RP::kC; m++) {
    const int c = j + kLpr * m;
    if (c >= nchunks) break;
    const u32x4 va = P.wa[m], vb = P.wb[m];
    if constexpr (DOT == kBF16) {
      const float4* xp = reinterpret_cast<const float4*>(xl + c * 8);
      const float4* yp = reinterpret_cast<const float4*>(xl + xb_off + c * 8);
      const float4 x0 = xp[0], x1 = xp[1], y0 = yp[0], y1 = yp[1];
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      const float yv[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        a0 = fmaf(bf16_lo(va[i]), xv[2 * i], a0);
        a0 = fmaf(bf16_hi(va[i]), xv[2 * i + 1], a0);
        a1 = fmaf(bf16_lo(vb[i]), yv[2 * i], a1);
        a1 = fmaf(bf16_hi(vb[i]), yv[2 * i + 1], a1);
      }
    } else if constexpr (DOT == kInt8) {
      // The chunk lies inside one 32-block, so its scale factors out: the
      // sixteen int8 * x products accumulate first (exact integers times x,
      // one conversion per byte), then one multiply-add by the block scale.
      // The reference rounds each dequantised weight first; the sums agree
      // to FP32 rounding.
      const float4* xp = reinterpret_cast<const float4*>(xl + c * 16);
      const float4* yp = reinterpret_cast<const float4*>(xl + xb_off + c * 16);
      float pa = 0.0f, pb = 0.0f;
#pragma unroll
      for (int v4 = 0; v4 < 4; v4++) {
        const float4 xv = xp[v4], yv = yp[v4];
        const float x4[4] = {xv.x, xv.y, xv.z, xv.w};
        const float y4[4] = {yv.x, yv.y, yv.z, yv.w};
#pragma unroll
        for (int b = 0; b < 4; b++) {
          pa = fmaf((float)(int8_t)((va[v4] >> (8 * b)) & 0xff), x4[b], pa);
          pb = fmaf((float)(int8_t)((vb[v4] >> (8 * b)) & 0xff), y4[b], pb);
        }
      }
      a0 = fmaf(pa, P.sa[m], a0);
      a1 = fmaf(pb, P.sb[m], a1);
    } else {
      const int4 xv = *reinterpret_cast<const int4*>(xq + c * 16);
      const int4 yv = *reinterpret_cast<const int4*>(xq + xb_off + c * 16);
      int pa = __builtin_amdgcn_sdot4((int)va.x, xv.x, 0, false);
      pa = __builtin_amdgcn_sdot4((int)va.y, xv.y, pa, false);
      pa = __builtin_amdgcn_sdot4((int)va.z, xv.z, pa, false);
      pa = __builtin_amdgcn_sdot4((int)va.w, xv.w, pa, false);
      int pb = __builtin_amdgcn_sdot4((int)vb.x, yv.x, 0, false);
      pb = __builtin_amdgcn_sdot4((int)vb.y, yv.y, pb, false);
      pb = __builtin_amdgcn_sdot4((int)vb.z, yv.z, pb, false);
      pb = __builtin_amdgcn_sdot4((int)vb.w, yv.w, pb, false);
      // Chunks 2b and 2b+1 (lanes j, j^1) form block b: exact i32 sum (the
      // partner's value by a DPP quad swap, no LDS round trip). Even lanes
      // add the block's scaled sum, odd lanes add zero: their partial sums
      // stay +0, as if they had skipped the block.
      const int ia = pa + __builtin_amdgcn_mov_dpp(pa, 0xB1, 0xf, 0xf, false);
      const int ib = pb + __builtin_amdgcn_mov_dpp(pb, 0xB1, 0xf, 0xf, false);
      const bool even = (j & 1) == 0;
      const int b = c >> 1;
      const float fa = (float)ia * P.sa[m] * xs[b];
      const float fb = (float)ib * P.sb[m] * xs[(xb_off >> 5) + b];
      a0 += even ? fa : 0.0f;
      a1 += even ? fb : 0.0f;
      if (even) {
        if (sums.a && b < sums.na) sums.a[b] = ia;
        if (sums.b && b < sums.nb) sums.b[b] = ib;
      }
    }
  }
  r0 = row16_sum(a0);
  r1 = row16_sum(a1);
}

template <int KIND, int KMAX>
__device__ __forceinline__ void dot_rows(const RowPair<KIND, KMAX>& P, int K, const float* xl,
                                         const int8_t* xq, const float* xs, float& r0,
                                         float& r1, const BlockSumOut& sums = BlockSumOut()) {
  dot_rows_as<KIND>(P, K, xl, xq, xs, r0, r1, 0, sums);
}

// An FP32 row of n <= N values (n % 4 == 0) held in registers of one wave
// (float4 at lane, lane + 64, ...): load_row issues every load (with buffer
// cache policy AUX), store_row writes the row into LDS.
template <int N>
struct RowStage {
  static constexpr int kV = N / 4 / 64;
  u32x4 v[kV];
};
template <int N, int AUX = 0>
__device__ __forceinline__ void load_row(RowStage<N>& R, const float* src, int n, int lane) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(src, (uint32_t)n * 4u);
#pragma unroll
  for (int i = 0; i < RowStage<N>::kV; i++) {
    const int at = lane + 64 * i;
    R.v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, at * 4 < n ? (uint32_t)at * 16u : kOut, 0, AUX);
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

// Dots both rows with NT activation rows held in LDS (row t at xl + t * ld;
// with SEG_B the b segment from element xb_off of the row), FP32
// (BF16 or INT8 weight-only kinds). a0[t] / a1[t] hold this lane's partial
// sums; row16_sum() completes them. Each chunk's weights are widened once
// and dotted with every token (straight-line code: NT is exact). BF16
// products accumulate in chunk order; INT8 chunks (inside one 32-block) sum
// q * x per token and apply the block scale once.
template <int KIND, int KMAX, int NT, bool SEG_B = false>
__device__ __forceinline__ void dot_rows_multi(const RowPair<KIND, KMAX>& P, int K, const float* xl,
                                               int xb_off, int ld, float (&a0)[NT],
                                               float (&a1)[NT]) {
  static_assert(KIND != kW8A8, "W8A8 groups are single-row: dot_rows");
  using RP = RowPair<KIND, KMAX>;
  constexpr int E = RP::kElems;
  const int j = threadIdx.x & (kLpr - 1);
  const int nchunks = K / E;
#pragma unroll
  for (int m = 0; m < RP::kC; m++) {
    const int c = j + kLpr * m;
    if (c >= nchunks) break;
    u32x4 va = P.wa[m], vb = P.wb[m];
    // Opaque copies keep the widening inside the caller's loops: hoisted
    // out of them, every chunk's widened weights would be live at once.
    asm volatile("" : "+v"(va), "+v"(vb));
    float wa[E], wb[E];
#pragma unroll
    for (int i = 0; i < E; i++) {
      if constexpr (KIND == kBF16) {
        wa[i] = (i & 1) ? bf16_hi(va[i >> 1]) : bf16_lo(va[i >> 1]);
        wb[i] = (i & 1) ? bf16_hi(vb[i >> 1]) : bf16_lo(vb[i >> 1]);
      } else {
        wa[i] = (float)(int8_t)((va[i >> 2] >> (8 * (i & 3))) & 0xff);
        wb[i] = (float)(int8_t)((vb[i >> 2] >> (8 * (i & 3))) & 0xff);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float4* xp = reinterpret_cast<const float4*>(xl + t * ld + c * E);
      float pa = KIND == kBF16 ? a0[t] : 0.0f, pb = KIND == kBF16 ? a1[t] : 0.0f;
      const float4* yp =
          reinterpret_cast<const float4*>(xl + t * ld + (SEG_B ? xb_off : 0) + c * E);
#pragma unroll
      for (int v4 = 0; v4 < E / 4; v4++) {
        const float4 xv = xp[v4], yv = yp[v4];
        pa = fmaf(wa[4 * v4 + 0], xv.x, pa);
        pa = fmaf(wa[4 * v4 + 1], xv.y, pa);
        pa = fmaf(wa[4 * v4 + 2], xv.z, pa);
        pa = fmaf(wa[4 * v4 + 3], xv.w, pa);
        pb = fmaf(wb[4 * v4 + 0], yv.x, pb);
        pb = fmaf(wb[4 * v4 + 1], yv.y, pb);
        pb = fmaf(wb[4 * v4 + 2], yv.z, pb);
        pb = fmaf(wb[4 * v4 + 3], yv.w, pb);
      }
      if constexpr (KIND == kBF16) {
        a0[t] = pa;
        a1[t] = pb;
      } else {
        a0[t] = fmaf(pa, P.sa[m], a0[t]);
        a1[t] = fmaf(pb, P.sb[m], a1[t]);
      }
      // One token's activations in registers at a time (the other waves
      // of the SIMD cover the LDS latency).
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Loads rows [0, n) of an FP32 [*, K] matrix, row t taken from src_rows[t]
// (K % 4 == 0), into LDS at dst + t * K with every thread of the workgroup;
// all loads of a thread are issued before its stores.
template <int PER_THREAD>
__device__ __forceinline__ void stage_rows_lds(const float* const* src_rows, int n, int K,
                                               float* dst) {
  const int vec = K / 4;
  const int total = n * vec;
  u32x4 v[PER_THREAD];
#pragma unroll
  for (int i = 0; i < PER_THREAD; i++) {
    const int at = threadIdx.x + i * blockDim.x;
    if (at < total) {
      const int t = at / vec, c = at - t * vec;
      v[i] = reinterpret_cast<const u32x4*>(src_rows[t])[c];
    }
  }
#pragma unroll
  for (int i = 0; i < PER_THREAD; i++) {
    const int at = threadIdx.x + i * blockDim.x;
    if (at < total) reinterpret_cast<u32x4*>(dst)[at] = v[i];
  }
}

}  // namespace uocr
