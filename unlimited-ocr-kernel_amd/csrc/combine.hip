// Ordered combine back to token order, and RMSNorm (fused into the combine
// when a following layer's norm is given).
//
// Combine: out[t] = shared(x)[t], then for t's experts in ascending id,
// out[t] += p * expert_out — one rounded multiply and one rounded add per
// term, as `*dest += probability * value` (src/decoder/mod.rs:185-194,
// 208-216). With a residual, out[t] = residual[t] + that (:361-363).
// Fixed order and no atomics: bit-reproducible run to run.
#include "common.hpp"
#include "moe_kernels.hpp"
#include "rownorm.hpp"

namespace uocr {

// Four consecutive values of an f32 row, or of a bf16 row (Y16).
template <bool Y16>
__device__ __forceinline__ float4 load4(const float* __restrict__ row, int i) {
  if constexpr (Y16) {
    const uint2 b = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(row) + i);
    return make_float4(__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xffff0000u),
                       __uint_as_float(b.y << 16), __uint_as_float(b.y & 0xffff0000u));
  } else {
    return *reinterpret_cast<const float4*>(row + i);
  }
}

// Combine, then (NORM) the next layer's RMSNorm of the result. Y16: the
// expert outputs (routed and shared) are bf16 rows (BF16 activations).
template <bool NORM, bool Y16>
__global__ __launch_bounds__(kRowThreads) void combine_kernel(
    const float* __restrict__ ys, const float* __restrict__ y, const int* __restrict__ ids,
    const float* __restrict__ w, const int* __restrict__ inv_pos, const float* __restrict__ residual,
    int H, int K, float* __restrict__ out, RowNorm nn, int* err) {
  const int t = blockIdx.x;
  int e[8], pos[8];
  float p[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    e[j] = j < K ? ids[(size_t)t * K + j] : 0x7fffffff;
    pos[j] = j < K ? inv_pos[(size_t)t * K + j] : 0;
    p[j] = j < K ? w[(size_t)t * K + j] : 0.0f;
  }
  // Ascending expert id (ids of one token are distinct).
#pragma unroll
  for (int a = 1; a < 8; a++) {
#pragma unroll
    for (int b = a; b > 0; b--) {
      if (e[b] < e[b - 1]) {
        int te = e[b]; e[b] = e[b - 1]; e[b - 1] = te;
        int tp = pos[b]; pos[b] = pos[b - 1]; pos[b - 1] = tp;
        float tw = p[b]; p[b] = p[b - 1]; p[b - 1] = tw;
      }
    }
  }
  // Every load of the row is issued before the first is used (the expert
  // rows of slots j >= K read slot 0's row again and are not used).
  const size_t rs = Y16 ? (size_t)H / 2 : (size_t)H;  // row stride in floats
  float4 sv[kRowChunks], rv[kRowChunks], v[kRowChunks][8];
#pragma unroll
  for (int it = 0; it < kRowChunks; it++) {
    const int i = (threadIdx.x + kRowThreads * it) * 4;
    if (i >= H) break;
    sv[it] = load4<Y16>(ys + t * rs, i);
#pragma unroll
    for (int j = 0; j < 8; j++) v[it][j] = load4<Y16>(y + (j < K ? pos[j] : pos[0]) * rs, i);
    if (residual) rv[it] = *reinterpret_cast<const float4*>(residual + (size_t)t * H + i);
  }
  float4 row[kRowChunks];
#pragma unroll
  for (int it = 0; it < kRowChunks; it++) {
    const int i = (threadIdx.x + kRowThreads * it) * 4;
    if (i >= H) break;
    float4 acc = sv[it];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (j < K) {
        const float4 u = v[it][j];
        acc.x = acc.x + p[j] * u.x;
        acc.y = acc.y + p[j] * u.y;
        acc.z = acc.z + p[j] * u.z;
        acc.w = acc.w + p[j] * u.w;
      }
    }
    if (residual) {
      const float4 r = rv[it];
      acc.x = r.x + acc.x;
      acc.y = r.y + acc.y;
      acc.z = r.z + acc.z;
      acc.w = r.w + acc.w;
    }
    *reinterpret_cast<float4*>(out + (size_t)t * H + i) = acc;
    row[it] = acc;
  }
  if constexpr (NORM)
    norm_row(row, H, nn.w, nn.eps, nn.out + (size_t)t * H, nn.hi, nn.lo, err, (int)gridDim.x, t);
}

// The same for rows up to kWaveRowWidth wide: one token per wave, four per
// workgroup, so a CU holds 8 rows' loads in flight instead of 5 (185
// VGPRs: two waves per SIMD; bounding them to three spills). At 4096
// tokens: fused FP32-class combine 45.4 -> 41.7 us, BF16 30.9 -> 28.2 us
// (rocprofv3, one box). Without a norm the forms give the same bits, and
// batches under kWaveMinTokens keep one token per workgroup (16 tokens:
// 4 workgroups would leave most CUs idle). KT: the number of experts per
// token when it is 6 (the model's), else 8 with slots j >= K reading
// slot 0's row again.
constexpr int kWaveMinTokens = 1024;
template <bool NORM, bool Y16, int KT>
__global__ __launch_bounds__(256) void combine_wave_kernel(
    const float* __restrict__ ys, const float* __restrict__ y, const int* __restrict__ ids,
    const float* __restrict__ w, const int* __restrict__ inv_pos, const float* __restrict__ residual,
    int H, int K, int T, float* __restrict__ out, RowNorm nn, int* err) {
  const int lane = threadIdx.x & 63;
  const int t = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
  if (t >= T) return;  // whole waves; no barrier below
  int e[KT], pos[KT];
  float p[KT];
#pragma unroll
  for (int j = 0; j < KT; j++) {
    e[j] = j < K ? ids[(size_t)t * K + j] : 0x7fffffff;
    pos[j] = j < K ? inv_pos[(size_t)t * K + j] : 0;
    p[j] = j < K ? w[(size_t)t * K + j] : 0.0f;
  }
  // Ascending expert id (ids of one token are distinct).
#pragma unroll
  for (int a = 1; a < KT; a++) {
#pragma unroll
    for (int b = a; b > 0; b--) {
      if (e[b] < e[b - 1]) {
        int te = e[b]; e[b] = e[b - 1]; e[b - 1] = te;
        int tp = pos[b]; pos[b] = pos[b - 1]; pos[b - 1] = tp;
        float tw = p[b]; p[b] = p[b - 1]; p[b - 1] = tw;
      }
    }
  }
  const size_t rs = Y16 ? (size_t)H / 2 : (size_t)H;  // row stride in floats
  float4 sv[kWaveChunks], rv[kWaveChunks], v[kWaveChunks][KT];
#pragma unroll
  for (int it = 0; it < kWaveChunks; it++) {
    const int i = (lane + 64 * it) * 4;
    if (i >= H) break;
    sv[it] = load4<Y16>(ys + t * rs, i);
#pragma unroll
    for (int j = 0; j < KT; j++) v[it][j] = load4<Y16>(y + (j < K ? pos[j] : pos[0]) * rs, i);
    if (residual) rv[it] = *reinterpret_cast<const float4*>(residual + (size_t)t * H + i);
  }
  float4 row[kWaveChunks];
#pragma unroll
  for (int it = 0; it < kWaveChunks; it++) {
    const int i = (lane + 64 * it) * 4;
    if (i >= H) break;
    float4 acc = sv[it];
#pragma unroll
    for (int j = 0; j < KT; j++) {
      if (j < K) {
        const float4 u = v[it][j];
        acc.x = acc.x + p[j] * u.x;
        acc.y = acc.y + p[j] * u.y;
        acc.z = acc.z + p[j] * u.z;
        acc.w = acc.w + p[j] * u.w;
      }
    }
    if (residual) {
      const float4 r = rv[it];
      acc.x = r.x + acc.x;
      acc.y = r.y + acc.y;
      acc.z = r.z + acc.z;
      acc.w = r.w + acc.w;
    }
    *reinterpret_cast<float4*>(out + (size_t)t * H + i) = acc;
    row[it] = acc;
  }
  if constexpr (NORM)
    norm_row_wave(row, H, nn.w, nn.eps, nn.out + (size_t)t * H, nn.hi, nn.lo, err, T, t, lane);
}

void launch_combine(const Scratch& S, const float* residual, int T, int H, int K, float* out,
                    const RowNorm* next, bool y16, hipStream_t s) {
  if (T <= 0) return;
  const RowNorm nn = next ? *next : RowNorm{};
  if (row_norm_wave(H) && K <= 8 && (next || T >= kWaveMinTokens)) {
    const dim3 grid((unsigned)((T + 3) / 4));
#define UOCR_COMBINE_WAVE(NORM, Y16)                                                          \
  do {                                                                                        \
    if (K == 6)                                                                               \
      combine_wave_kernel<NORM, Y16, 6><<<grid, 256, 0, s>>>(                                 \
          S.ys, S.y, S.topk_ids, S.topk_w, S.inv_pos, residual, H, K, T, out, nn, S.err);      \
    else                                                                                      \
      combine_wave_kernel<NORM, Y16, 8><<<grid, 256, 0, s>>>(                                 \
          S.ys, S.y, S.topk_ids, S.topk_w, S.inv_pos, residual, H, K, T, out, nn, S.err);      \
  } while (0)
    if (next && y16)
      UOCR_COMBINE_WAVE(true, true);
    else if (next)
      UOCR_COMBINE_WAVE(true, false);
    else if (y16)
      UOCR_COMBINE_WAVE(false, true);
    else
      UOCR_COMBINE_WAVE(false, false);
#undef UOCR_COMBINE_WAVE
    return;
  }
#define UOCR_COMBINE(NORM, Y16)                                                               \
  combine_kernel<NORM, Y16><<<T, kRowThreads, 0, s>>>(S.ys, S.y, S.topk_ids, S.topk_w,         \
                                                      S.inv_pos, residual, H, K, out, nn, S.err)
  if (next && y16)
    UOCR_COMBINE(true, true);
  else if (next)
    UOCR_COMBINE(true, false);
  else if (y16)
    UOCR_COMBINE(false, true);
  else
    UOCR_COMBINE(false, false);
#undef UOCR_COMBINE
}

__global__ __launch_bounds__(kRowThreads) void rms_norm_kernel(const float* __restrict__ x, int width,
                                                               RowNorm nn, int* err) {
  const int t = blockIdx.x;
  float4 row[kRowChunks];
#pragma unroll
  for (int it = 0; it < kRowChunks; it++) {
    const int i = (threadIdx.x + kRowThreads * it) * 4;
    if (i >= width) break;
    row[it] = *reinterpret_cast<const float4*>(x + (size_t)t * width + i);
  }
  norm_row(row, width, nn.w, nn.eps, nn.out + (size_t)t * width, nn.hi, nn.lo, err, (int)gridDim.x,
           t);
}

// Rows up to kWaveRowWidth wide: one row per wave, four per workgroup, the
// fused norm's form (4096 x 1280: 14.3 -> 12.4 us).
__global__ __launch_bounds__(256) void rms_norm_wave_kernel(const float* __restrict__ x, int rows,
                                                            int width, RowNorm nn, int* err) {
  const int lane = threadIdx.x & 63;
  const int t = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
  if (t >= rows) return;
  float4 row[kWaveChunks];
#pragma unroll
  for (int it = 0; it < kWaveChunks; it++) {
    const int i = (lane + 64 * it) * 4;
    if (i >= width) break;
    row[it] = *reinterpret_cast<const float4*>(x + (size_t)t * width + i);
  }
  norm_row_wave(row, width, nn.w, nn.eps, nn.out + (size_t)t * width, nn.hi, nn.lo, err, rows, t,
                lane);
}

// Wider rows: one workgroup per row, scalar passes.
__global__ __launch_bounds__(256) void rms_norm_wide_kernel(const float* __restrict__ x, int width,
                                                            const float* __restrict__ w, float eps,
                                                            float* __restrict__ out, int* err) {
  __shared__ float partial[4];
  __shared__ int bad_any;
  const int row = blockIdx.x;
  const float* in = x + (size_t)row * width;
  if (threadIdx.x == 0) bad_any = 0;
  __syncthreads();
  float ss = 0.0f;
  bool bad = false;
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    const float v = in[i];
    bad |= !isfinite(v) || !isfinite(w[i]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  if (bad) bad_any = 1;
  __syncthreads();
  const float total = partial[0] + partial[1] + partial[2] + partial[3];
  if (bad_any) {
    if (threadIdx.x == 0) raise_error(err, kErrNumerical);
  }
  const float variance = total / (float)width;
  const float scale = 1.0f / sqrtf(variance + eps);
  for (int i = threadIdx.x; i < width; i += blockDim.x) out[(size_t)row * width + i] = in[i] * scale * w[i];
}

bool row_norm_fusable(int width) { return width % 4 == 0 && width <= kRowThreads * kRowChunks * 4; }
bool row_norm_wave(int width) { return width % 4 == 0 && width <= kWaveRowWidth; }

void launch_rms_norm(const float* x, int rows, int width, const RowNorm& nn, int* err,
                     hipStream_t s) {
  if (rows <= 0) return;
  if (row_norm_wave(width))
    rms_norm_wave_kernel<<<(rows + 3) / 4, 256, 0, s>>>(x, rows, width, nn, err);
  else if (row_norm_fusable(width))
    rms_norm_kernel<<<rows, kRowThreads, 0, s>>>(x, width, nn, err);
  else
    rms_norm_wide_kernel<<<rows, 256, 0, s>>>(x, width, nn.w, nn.eps, nn.out, err);
}

}  // namespace uocr
