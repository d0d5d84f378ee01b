// Row-chunk expert engine: streams each active expert matrix once per chunk
// of up to NMAX tokens and computes in FP32 on the vector ALUs. Used for
// decode (one token) and small batches, where the layer is bound by the
// bytes of the active experts' weights.
//
// Arithmetic follows Decoder::projection (src/decoder/mod.rs:99-112):
//  - BF16 weights: exact widening (src/checkpoint.rs:79-85), FP32 dot
//    (src/cpu/ops.rs:84-118);
//  - INT8 weight-only: each weight dequantised as the rounded product
//    w * scale, then dotted in FP32 (src/cpu/quantized.rs:119-131);
//  - W8A8 (DynamicActivations and a single-row group, :103-104): the row is
//    quantised per 32-block (src/cpu/quantized.rs:43-74), each block's
//    int8 x int8 sum is an exact i32 (v_dot4_i32_i8), then
//    (sum as f32 * w_scale) * x_scale is accumulated (:190-198).
// Only the order of the FP32 accumulation differs from the reference.
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {

enum { kKindBF16 = 0, kKindInt8 = 1, kKindW8A8 = 2 };

// Quantise one FP32 row held in LDS per 32-element block (K % 32 == 0):
// absmax/127 scale, round-half-even, clamp to +-127. Non-finite input or an
// underflowing scale raises Numerical, like Int8Matrix::quantize.
__device__ void quantize_row_lds(const float* xl, int K, int8_t* xq, float* xs, int* err) {
  const int nblk = K / kQBlock;
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    const float* v = xl + b * kQBlock;
    float maximum = 0.0f;
    bool bad = false;
    for (int i = 0; i < kQBlock; i++) {
      bad |= !isfinite(v[i]);
      maximum = fmaxf(maximum, fabsf(v[i]));
    }
    float scale = maximum / 127.0f;
    if (bad || (maximum > 0.0f && scale == 0.0f)) raise_error(err, kErrNumerical);
    xs[b] = scale;
    for (int i = 0; i < kQBlock; i++) {
      int q = 0;
      if (scale != 0.0f) {
        float r = rintf(v[i] / scale);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        q = (int)r;
      }
      xq[b * kQBlock + i] = (int8_t)q;
    }
  }
}

// 64 consecutive rows [row_begin, row_begin + 64) of a [rows_total, K]
// matrix against n <= NMAX activation rows in LDS. 16 lanes share a row;
// lane j reads 16-byte chunks j, j+16, ... of it. out[r * NMAX + m] receives
// the dot of row r with activation m. K % 64 == 0.
template <int KIND, int NMAX>
__device__ __forceinline__ void gemv_rows64(const void* __restrict__ wbase,
                                            const float* __restrict__ sbase, int K,
                                            int rows_total, int row_begin,
                                            const float* __restrict__ xl, int n,
                                            const int8_t* __restrict__ xq,
                                            const float* __restrict__ xqs, float* out,
                                            int32_t* __restrict__ block_sums) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q = lane >> 4;
  const int j = lane & 15;
  constexpr int kElems = KIND == kKindBF16 ? 8 : 16;
  constexpr int kBytes = KIND == kKindBF16 ? 2 : 1;
  const int nchunks = K / kElems;
  const int nblk = K / kQBlock;
#pragma unroll 1
  for (int it = 0; it < 4; it++) {
    const int r = wave * 16 + it * 4 + q;
    const int row = row_begin + r;
    float acc[NMAX];
#pragma unroll
    for (int m = 0; m < NMAX; m++) acc[m] = 0.0f;
    if (row < rows_total) {
      const uint4* wrow =
          reinterpret_cast<const uint4*>(static_cast<const char*>(wbase) + (size_t)row * K * kBytes);
      for (int c = j; c < nchunks; c += 16) {
        const uint4 wv = wrow[c];
        if constexpr (KIND == kKindBF16) {
          const float wf[8] = {bf16_lo(wv.x), bf16_hi(wv.x), bf16_lo(wv.y), bf16_hi(wv.y),
                               bf16_lo(wv.z), bf16_hi(wv.z), bf16_lo(wv.w), bf16_hi(wv.w)};
#pragma unroll
          for (int m = 0; m < NMAX; m++) {
            if (m < n) {
              const float4* xp = reinterpret_cast<const float4*>(xl + (size_t)m * K + c * 8);
              const float4 x0 = xp[0], x1 = xp[1];
              float a = acc[m];
              a = fmaf(wf[0], x0.x, a);
              a = fmaf(wf[1], x0.y, a);
              a = fmaf(wf[2], x0.z, a);
              a = fmaf(wf[3], x0.w, a);
              a = fmaf(wf[4], x1.x, a);
              a = fmaf(wf[5], x1.y, a);
              a = fmaf(wf[6], x1.z, a);
              a = fmaf(wf[7], x1.w, a);
              acc[m] = a;
            }
          }
        } else if constexpr (KIND == kKindInt8) {
          const float s = sbase[(size_t)row * nblk + (c >> 1)];
          const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
          float d[16];
#pragma unroll
          for (int i = 0; i < 16; i++) {
            const int8_t v = (int8_t)((words[i >> 2] >> (8 * (i & 3))) & 0xff);
            d[i] = (float)v * s;  // the dequantised weight, rounded once
          }
#pragma unroll
          for (int m = 0; m < NMAX; m++) {
            if (m < n) {
              const float4* xp = reinterpret_cast<const float4*>(xl + (size_t)m * K + c * 16);
              float a = acc[m];
#pragma unroll
              for (int v4 = 0; v4 < 4; v4++) {
                const float4 xv = xp[v4];
                a = fmaf(d[4 * v4 + 0], xv.x, a);
                a = fmaf(d[4 * v4 + 1], xv.y, a);
                a = fmaf(d[4 * v4 + 2], xv.z, a);
                a = fmaf(d[4 * v4 + 3], xv.w, a);
              }
              acc[m] = a;
            }
          }
        } else {
          const int4 xv = *reinterpret_cast<const int4*>(xq + c * 16);
          int part = __builtin_amdgcn_sdot4((int)wv.x, xv.x, 0, false);
          part = __builtin_amdgcn_sdot4((int)wv.y, xv.y, part, false);
          part = __builtin_amdgcn_sdot4((int)wv.z, xv.z, part, false);
          part = __builtin_amdgcn_sdot4((int)wv.w, xv.w, part, false);
          // Chunks 2b and 2b+1 form block b and sit in lanes j and j^1.
          const int sum = part + __shfl_xor(part, 1);
          if ((j & 1) == 0) {
            const int b = c >> 1;
            if (block_sums) block_sums[(size_t)row * nblk + b] = sum;
            const float f = (float)sum * sbase[(size_t)row * nblk + b] * xqs[b];
            acc[0] += f;
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < NMAX; m++) {
      const float v = group16_sum(acc[m]);
      if (j == 0 && row < rows_total && m < n) out[r * NMAX + m] = v;
    }
  }
}

struct GemvLds {
  float* xl;      // [NMAX, Kmax]
  float* out;     // [64, NMAX]
  int8_t* xq;     // [Kmax], 16-byte aligned
  float* xqs;     // [Kmax / 32]
};

template <int NMAX>
__device__ GemvLds carve_lds(char* smem, int kmax) {
  GemvLds l;
  l.xl = reinterpret_cast<float*>(smem);
  l.out = l.xl + (size_t)NMAX * kmax;
  l.xq = reinterpret_cast<int8_t*>(l.out + 64 * NMAX);
  l.xqs = reinterpret_cast<float*>(l.xq + kmax);
  return l;
}

static size_t gemv_lds_bytes(int nmax, int kmax) {
  return (size_t)nmax * kmax * 4 + 64 * nmax * 4 + (kmax / kQBlock) * 4 + kmax;
}

// Loads n activation rows (row index from `rows`, or r0 + m when rows is
// null) of a [*, K] FP32 matrix into LDS.
__device__ void stage_rows(const float* __restrict__ src, const int* __restrict__ rows, int r0,
                           int n, int K, float* xl) {
  const int vec = K / 4;
  for (int i = threadIdx.x; i < n * vec; i += blockDim.x) {
    const int m = i / vec, v = i % vec;
    const int row = rows ? rows[r0 + m] : r0 + m;
    reinterpret_cast<float4*>(xl + (size_t)m * K)[v] =
        reinterpret_cast<const float4*>(src + (size_t)row * K)[v];
  }
}

// ------------------------------------------------------------- operators
// Single-matrix entry points. Column counts that are multiples of 64 use the
// same row engine as the layer; other widths take a plain per-element path.

template <int KIND>
__global__ __launch_bounds__(256) void op_gemv_kernel(const void* w, const float* sc, int rows,
                                                      int K, const float* x, int m_total,
                                                      float* y, int32_t* block_sums, int* err) {
  extern __shared__ __align__(16) char smem[];
  constexpr int NM = KIND == kKindW8A8 ? 1 : kGemvChunk;
  GemvLds l = carve_lds<NM>(smem, K);
  const int m0 = blockIdx.y * NM;
  const int n = min(NM, m_total - m0);
  stage_rows(x, nullptr, m0, n, K, l.xl);
  __syncthreads();
  if (KIND == kKindW8A8) {
    quantize_row_lds(l.xl, K, l.xq, l.xqs, err);
    __syncthreads();
  }
  gemv_rows64<KIND, NM>(w, sc, K, rows, blockIdx.x * 64, l.xl, n, l.xq, l.xqs, l.out, block_sums);
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * n; i += blockDim.x) {
    const int r = i & 63, m = i >> 6;
    const int row = blockIdx.x * 64 + r;
    if (row < rows) y[(size_t)(m0 + m) * rows + row] = l.out[r * NM + m];
  }
}

// Any width: one wave per output element.
template <int KIND>
__global__ __launch_bounds__(256) void op_generic_kernel(const void* w, const float* sc, int rows,
                                                         int K, const float* x, int m_total,
                                                         float* y) {
  const int lane = threadIdx.x & 63;
  const long long out = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (out >= (long long)rows * m_total) return;
  const int m = (int)(out / rows), row = (int)(out % rows);
  const int nblk = (K + kQBlock - 1) / kQBlock;
  float acc = 0.0f;
  for (int k = lane; k < K; k += 64) {
    float wv;
    if (KIND == kKindBF16) {
      wv = __uint_as_float((uint32_t)static_cast<const uint16_t*>(w)[(size_t)row * K + k] << 16);
    } else {
      wv = (float)static_cast<const int8_t*>(w)[(size_t)row * K + k] *
           sc[(size_t)row * nblk + k / kQBlock];
    }
    acc = fmaf(wv, x[(size_t)m * K + k], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[(size_t)m * rows + row] = acc;
}

void launch_linear_bf16(const float* x, int m, int k, const uint16_t* w, int n, float* y,
                        hipStream_t s) {
  if (m <= 0 || n <= 0) return;
  if (k % 64 == 0) {
    dim3 grid((n + 63) / 64, (m + kGemvChunk - 1) / kGemvChunk);
    hipLaunchKernelGGL(op_gemv_kernel<kKindBF16>, grid, dim3(256), gemv_lds_bytes(kGemvChunk, k),
                       s, (const void*)w, (const float*)nullptr, n, k, x, m, y,
                       (int32_t*)nullptr, (int*)nullptr);
  } else {
    long long outs = (long long)m * n;
    hipLaunchKernelGGL(op_generic_kernel<kKindBF16>, dim3((unsigned)((outs + 3) / 4)), dim3(256),
                       0, s, (const void*)w, (const float*)nullptr, n, k, x, m, y);
  }
}

void launch_int8_linear(const int8_t* q, const float* sc, int rows, int cols, const float* x,
                        int batch, float* y, hipStream_t s) {
  if (batch <= 0 || rows <= 0) return;
  if (cols % 64 == 0) {
    dim3 grid((rows + 63) / 64, (batch + kGemvChunk - 1) / kGemvChunk);
    hipLaunchKernelGGL(op_gemv_kernel<kKindInt8>, grid, dim3(256),
                       gemv_lds_bytes(kGemvChunk, cols), s, (const void*)q, sc, rows, cols, x,
                       batch, y, (int32_t*)nullptr, (int*)nullptr);
  } else {
    long long outs = (long long)batch * rows;
    hipLaunchKernelGGL(op_generic_kernel<kKindInt8>, dim3((unsigned)((outs + 3) / 4)), dim3(256),
                       0, s, (const void*)q, sc, rows, cols, x, batch, y);
  }
}

// Ragged-width W8A8: quantise the row per block in one pass, then one wave
// per output row, lane = block (exact i32 block sums).
__global__ void quantize_row_kernel(const float* x, int K, int8_t* xq, float* xs, int* err) {
  const int nblk = (K + kQBlock - 1) / kQBlock;
  for (int b = blockIdx.x * blockDim.x + threadIdx.x; b < nblk; b += gridDim.x * blockDim.x) {
    const int start = b * kQBlock, end = min(start + kQBlock, K);
    float maximum = 0.0f;
    bool bad = false;
    for (int i = start; i < end; i++) {
      bad |= !isfinite(x[i]);
      maximum = fmaxf(maximum, fabsf(x[i]));
    }
    const float scale = maximum / 127.0f;
    if (bad || (maximum > 0.0f && scale == 0.0f)) raise_error(err, kErrNumerical);
    xs[b] = scale;
    for (int i = start; i < end; i++) {
      int q = 0;
      if (scale != 0.0f) q = (int)fminf(fmaxf(rintf(x[i] / scale), -127.0f), 127.0f);
      xq[i] = (int8_t)q;
    }
  }
}

__global__ __launch_bounds__(256) void dynamic_generic_kernel(const int8_t* q, const float* sc,
                                                              int rows, int K,
                                                              const int8_t* xq, const float* xs,
                                                              float* y, int32_t* block_sums) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nblk = (K + kQBlock - 1) / kQBlock;
  float acc = 0.0f;
  for (int b = lane; b < nblk; b += 64) {
    const int start = b * kQBlock, end = min(start + kQBlock, K);
    int sum = 0;
    for (int i = start; i < end; i++) sum += (int)q[(size_t)row * K + i] * (int)xq[i];
    if (block_sums) block_sums[(size_t)row * nblk + b] = sum;
    const float f = (float)sum * sc[(size_t)row * nblk + b] * xs[b];
    acc += f;
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

void launch_int8_dynamic(const int8_t* q, const float* sc, int rows, int cols, const float* x,
                         float* y, int32_t* block_sums, int8_t* xq, float* xs, int* err,
                         hipStream_t s) {
  if (rows <= 0) return;
  if (cols % 64 == 0) {
    dim3 grid((rows + 63) / 64, 1);
    hipLaunchKernelGGL(op_gemv_kernel<kKindW8A8>, grid, dim3(256), gemv_lds_bytes(1, cols), s,
                       (const void*)q, sc, rows, cols, x, 1, y, block_sums, err);
  } else {
    // Ragged width: xq [cols] and xs [ceil(cols/32)] are caller scratch.
    const int nblk = (cols + kQBlock - 1) / kQBlock;
    hipLaunchKernelGGL(quantize_row_kernel, dim3((nblk + 255) / 256), dim3(256), 0, s, x, cols,
                       xq, xs, err);
    hipLaunchKernelGGL(dynamic_generic_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, q, sc, rows,
                       cols, xq, xs, y, block_sums);
  }
}

// Kernels whose dynamic LDS may exceed the 64 KiB default opt in once.
void gemv_init_attributes() {
  // Largest dynamic LDS any launch here asks for is gemv_lds_bytes(16, 1792)
  // = 118 KiB; static LDS plus this must stay within the 160 KiB per CU.
  const int big = 128 * 1024;
  (void)hipFuncSetAttribute((const void*)op_gemv_kernel<kKindBF16>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, big);
  (void)hipFuncSetAttribute((const void*)op_gemv_kernel<kKindInt8>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, big);
  (void)hipFuncSetAttribute((const void*)op_gemv_kernel<kKindW8A8>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, big);
  (void)hipGetLastError();  // a refused attribute surfaces at launch instead
}

}  // namespace uocr
