// Ordered combine back to token order, and RMSNorm.
//
// Combine: out[t] = shared(x)[t], then for t's experts in ascending id,
// out[t] += p * expert_out — one rounded multiply and one rounded add per
// term, as `*dest += probability * value` (src/decoder/mod.rs:185-194,
// 208-216). With a residual, out[t] = residual[t] + that (:361-363).
// Fixed order and no atomics: bit-reproducible run to run.
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ ys,
                                                      const float* __restrict__ y,
                                                      const int* __restrict__ ids,
                                                      const float* __restrict__ w,
                                                      const int* __restrict__ inv_pos,
                                                      const float* __restrict__ residual, int H,
                                                      int K, float* __restrict__ out) {
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
  for (int i = threadIdx.x * 4; i < H; i += blockDim.x * 4) {
    float4 acc = *reinterpret_cast<const float4*>(ys + (size_t)t * H + i);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (j < K) {
        const float4 v = *reinterpret_cast<const float4*>(y + (size_t)pos[j] * H + i);
        acc.x = acc.x + p[j] * v.x;
        acc.y = acc.y + p[j] * v.y;
        acc.z = acc.z + p[j] * v.z;
        acc.w = acc.w + p[j] * v.w;
      }
    }
    if (residual) {
      const float4 r = *reinterpret_cast<const float4*>(residual + (size_t)t * H + i);
      acc.x = r.x + acc.x;
      acc.y = r.y + acc.y;
      acc.z = r.z + acc.z;
      acc.w = r.w + acc.w;
    }
    *reinterpret_cast<float4*>(out + (size_t)t * H + i) = acc;
  }
}

void launch_combine(const Scratch& S, const float* residual, int T, int H, int K, float* out,
                    hipStream_t s) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(256), 0, s, S.ys, S.y, S.topk_ids, S.topk_w,
                     S.inv_pos, residual, H, K, out);
}

// RMSNorm (src/cpu/ops.rs:362-423, center = false): variance = sum(v^2)/W,
// scale = 1/sqrt(variance + eps), out = v * scale * w. Non-finite input ->
// Numerical (:382-389). One workgroup per row.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, int width,
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

void launch_rms_norm(const float* x, int rows, int width, const float* w, float eps, float* out,
                     int* err, hipStream_t s) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, s, x, width, w, eps, out, err);
}

}  // namespace uocr
