// RMSNorm of one row held by a workgroup of 256 threads (thread i holds
// float4 chunks i and i + 256: widths up to 2048), or by one wave (widths
// up to 1280). The combine and the standalone norm take the same form for
// a given width, so that a fused norm gives the standalone norm's bits;
// the vocabulary projection normalises its one row with the workgroup form.
#pragma once

#include "common.hpp"

namespace uocr {

// One row (token) per workgroup of 256 threads; thread i holds float4
// chunks i and i + 256 of the row (widths up to 2048).
constexpr int kRowThreads = 256, kRowChunks = 2;

// RMSNorm of a row held as float4 chunks (src/cpu/ops.rs:362-423, center =
// false): variance = sum(v^2) / W, scale = 1 / sqrt(variance + eps),
// out = v * scale * w. Non-finite row or weight -> Numerical (:382-389).
// The sum runs per thread over its chunks (x, y, z, w in turn), then over
// the wave and the four waves in order, so the standalone and the fused
// norms of a row wider than kWaveRowWidth give the same bits. Writes the normalised row and, when hi is set,
// its bf16 planes (hi = bf16(v), lo = bf16(v - hi) when lo is set): row t
// of `rows` into planes laid out [width/32][rows][32], as the MFMA engine
// reads them (hi / lo are the planes' bases).
__device__ inline void norm_row(const float4 (&v)[kRowChunks], int width, const float* __restrict__ w,
                                float eps, float* __restrict__ out, uint16_t* __restrict__ hi,
                                uint16_t* __restrict__ lo, int* err, int rows = 0, int t = 0) {
  __shared__ float partial[kRowThreads / 64];
  __shared__ int bad_any;
  const int tid = threadIdx.x;
  if (tid == 0) bad_any = 0;
  __syncthreads();
  float ss = 0.0f;
  bool bad = false;
  float4 wv[kRowChunks];
#pragma unroll
  for (int it = 0; it < kRowChunks; it++) {
    const int i = (tid + kRowThreads * it) * 4;
    if (i >= width) break;
    wv[it] = *reinterpret_cast<const float4*>(w + i);
    const float4 x = v[it];
    bad |= !isfinite(x.x) || !isfinite(x.y) || !isfinite(x.z) || !isfinite(x.w);
    bad |= !isfinite(wv[it].x) || !isfinite(wv[it].y) || !isfinite(wv[it].z) || !isfinite(wv[it].w);
    ss = fmaf(x.x, x.x, ss);
    ss = fmaf(x.y, x.y, ss);
    ss = fmaf(x.z, x.z, ss);
    ss = fmaf(x.w, x.w, ss);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) partial[tid >> 6] = ss;
  if (bad) bad_any = 1;
  __syncthreads();
  const float total = partial[0] + partial[1] + partial[2] + partial[3];
  if (bad_any && tid == 0) raise_error(err, kErrNumerical);
  const float scale = 1.0f / sqrtf(total / (float)width + eps);
#pragma unroll
  for (int it = 0; it < kRowChunks; it++) {
    const int i = (tid + kRowThreads * it) * 4;
    if (i >= width) break;
    const float4 x = v[it];
    const float o[4] = {x.x * scale * wv[it].x, x.y * scale * wv[it].y, x.z * scale * wv[it].z,
                        x.w * scale * wv[it].w};
    *reinterpret_cast<float4*>(out + i) = make_float4(o[0], o[1], o[2], o[3]);
    if (hi) {
      const size_t p = ((size_t)(i / 32) * rows + t) * 32 + i % 32;
      uint16_t h[4], l[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        h[j] = __builtin_bit_cast(uint16_t, (__bf16)o[j]);
        l[j] = __builtin_bit_cast(uint16_t, (__bf16)(o[j] - __uint_as_float((uint32_t)h[j] << 16)));
      }
      *reinterpret_cast<uint2*>(hi + p) =
          make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
      if (lo)
        *reinterpret_cast<uint2*>(lo + p) =
            make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    }
  }
}

// Rows up to kWaveRowWidth wide are held by one wave instead (lane l:
// float4 chunks l, l + 64, ...; kWaveChunks per lane), so that a
// workgroup of 256 threads works on four rows: the combine then keeps more
// rows in flight per CU, and the norm reduces inside the wave (per lane
// over its chunks, x, y, z, w in turn, then over the wave). The combine
// and the standalone norm take the same form for the same width, so a
// fused norm gives the standalone norm's bits.
constexpr int kWaveChunks = 5, kWaveRowWidth = 64 * 4 * kWaveChunks;  // 1280

__device__ inline void norm_row_wave(const float4 (&v)[kWaveChunks], int width,
                                     const float* __restrict__ w, float eps, float* __restrict__ out,
                                     uint16_t* __restrict__ hi, uint16_t* __restrict__ lo, int* err,
                                     int rows, int t, int lane) {
  float ss = 0.0f;
  bool bad = false;
  float4 wv[kWaveChunks];
#pragma unroll
  for (int it = 0; it < kWaveChunks; it++) {
    const int i = (lane + 64 * it) * 4;
    if (i >= width) break;
    wv[it] = *reinterpret_cast<const float4*>(w + i);
    const float4 x = v[it];
    bad |= !isfinite(x.x) || !isfinite(x.y) || !isfinite(x.z) || !isfinite(x.w);
    bad |= !isfinite(wv[it].x) || !isfinite(wv[it].y) || !isfinite(wv[it].z) || !isfinite(wv[it].w);
    ss = fmaf(x.x, x.x, ss);
    ss = fmaf(x.y, x.y, ss);
    ss = fmaf(x.z, x.z, ss);
    ss = fmaf(x.w, x.w, ss);
  }
  const float total = wave_sum(ss);
  if (__ballot(bad) != 0ull && lane == 0) raise_error(err, kErrNumerical);
  const float scale = 1.0f / sqrtf(total / (float)width + eps);
#pragma unroll
  for (int it = 0; it < kWaveChunks; it++) {
    const int i = (lane + 64 * it) * 4;
    if (i >= width) break;
    const float4 x = v[it];
    const float o[4] = {x.x * scale * wv[it].x, x.y * scale * wv[it].y, x.z * scale * wv[it].z,
                        x.w * scale * wv[it].w};
    *reinterpret_cast<float4*>(out + i) = make_float4(o[0], o[1], o[2], o[3]);
    if (hi) {
      const size_t p = ((size_t)(i / 32) * rows + t) * 32 + i % 32;
      uint16_t h[4], l[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        h[j] = __builtin_bit_cast(uint16_t, (__bf16)o[j]);
        l[j] = __builtin_bit_cast(uint16_t, (__bf16)(o[j] - __uint_as_float((uint32_t)h[j] << 16)));
      }
      *reinterpret_cast<uint2*>(hi + p) =
          make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
      if (lo)
        *reinterpret_cast<uint2*>(lo + p) =
            make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    }
  }
}

}  // namespace uocr
