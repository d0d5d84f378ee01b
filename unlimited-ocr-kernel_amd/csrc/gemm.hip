// MFMA grouped GEMM engine for multi-token batches (prefill), BF16 weights.
//
// Reference roles: the per-expert GEMMs of Decoder::experts / feed_forward
// (src/decoder/mod.rs:114-122, 197-218), which the reference runs as
// widened-FP32 scalar GEMMs (src/cpu/ops.rs:39-47, 119-132).
//
// One workgroup (4 waves, 2x2) computes a 128x128 output tile of one
// expert group with v_mfma_f32_32x32x16_bf16; each wave owns 64x64 (2x2
// MFMA tiles). Weights are exact in bf16. FP32 activations enter as bf16
// planes: with FP32-class precision each value is split x = hi + lo (two
// bf16, relative residual <= 2^-18) and both planes are multiplied; with
// BF16 activations only hi is used.
//
// Gate/up rows are interleaved in blocks of 32 (gate j.., up j..), so the
// wave whose 64 columns are one (gate, up) block pair holds g and u for the
// same (row, column) in the same lane and register: the SiLU(g) * u
// epilogue is register-local and h leaves as bf16 planes for the down GEMM.
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdsStride = kBK + 8;  // bf16 per LDS row (16-byte pad)

__device__ __forceinline__ uint16_t bf16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (__bf16)v);
}

// Split FP32 activations [rows, K] into bf16 hi and lo planes.
__global__ void split_planes_kernel(const float* __restrict__ x, size_t n,
                                    uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  const float4 v = *reinterpret_cast<const float4*>(x + i);
  const float f[4] = {v.x, v.y, v.z, v.w};
  uint16_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    h[j] = bf16_bits(f[j]);
    l[j] = bf16_bits(f[j] - __uint_as_float((uint32_t)h[j] << 16));
  }
  *reinterpret_cast<uint2*>(hi + i) =
      make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
  if (lo)
    *reinterpret_cast<uint2*>(lo + i) =
        make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
}

template <bool SPLIT, bool GATEUP>
__global__ __launch_bounds__(256) void mfma_group_kernel(DeviceLayer L, Scratch S, MfmaPlanes P,
                                                         int T) {
  __shared__ __align__(16) uint16_t as_hi[kBM * kLdsStride];
  __shared__ __align__(16) uint16_t as_lo[SPLIT ? kBM * kLdsStride : 8];
  __shared__ __align__(16) uint16_t bs[kBN * kLdsStride];
  __shared__ int arow[kBM];

  const int tile = blockIdx.y;
  if (tile >= S.counters[0]) return;
  const int g = S.tiles[2 * tile], r0 = S.tiles[2 * tile + 1];
  const bool routed = g < L.E;
  const int W = L.width(g);
  const int N = GATEUP ? 2 * W : L.H;
  const int K = GATEUP ? L.H : W;
  const int n0 = blockIdx.x * kBN;
  if (n0 >= N) return;
  const int group_rows = routed ? S.offsets[g + 1] - S.offsets[g] : T;
  const int mrows = min(kBM, group_rows - r0);
  const int base = routed ? S.offsets[g] : 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Source row of each local A row (-1 = padding).
  if (tid < kBM) {
    int src = -1;
    if (tid < mrows) {
      if (GATEUP)
        src = routed ? S.perm_rows[base + r0 + tid] : r0 + tid;
      else
        src = base + r0 + tid;
    }
    arow[tid] = src;
  }
  __syncthreads();

  const uint16_t* a_hi_src;
  const uint16_t* a_lo_src;
  if (GATEUP) {
    a_hi_src = P.x_hi;
    a_lo_src = P.x_lo;
  } else {
    a_hi_src = routed ? P.h_hi : P.hs_hi;
    a_lo_src = routed ? P.h_lo : P.hs_lo;
  }
  const uint16_t* wmat = GATEUP ? L.w13 + L.w13_offset(g) : L.w2 + L.w2_offset(g);

  // Global -> register mapping: thread covers row tid/2, k half (tid&1)*32.
  const int lrow = tid >> 1;
  const int lk = (tid & 1) * 32;
  const int src_row = arow[lrow];
  const bool brow_ok = n0 + lrow < N;
  const uint4* a_hi_ptr =
      src_row >= 0 ? reinterpret_cast<const uint4*>(a_hi_src + (size_t)src_row * K + lk) : nullptr;
  const uint4* a_lo_ptr = (SPLIT && src_row >= 0)
                              ? reinterpret_cast<const uint4*>(a_lo_src + (size_t)src_row * K + lk)
                              : nullptr;
  const uint4* b_ptr =
      brow_ok ? reinterpret_cast<const uint4*>(wmat + (size_t)(n0 + lrow) * K + lk) : nullptr;

  uint4 ra_hi[4], ra_lo[4], rb[4];
  const uint4 zero = make_uint4(0, 0, 0, 0);
  auto load_regs = [&](int k0) {
    const int off = k0 / 8;  // uint4 units
#pragma unroll
    for (int i = 0; i < 4; i++) {
      ra_hi[i] = a_hi_ptr ? a_hi_ptr[off + i] : zero;
      if (SPLIT) ra_lo[i] = a_lo_ptr ? a_lo_ptr[off + i] : zero;
      rb[i] = b_ptr ? b_ptr[off + i] : zero;
    }
  };
  auto store_lds = [&]() {
    uint4* dh = reinterpret_cast<uint4*>(as_hi + lrow * kLdsStride + lk);
    uint4* db = reinterpret_cast<uint4*>(bs + lrow * kLdsStride + lk);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      dh[i] = ra_hi[i];
      db[i] = rb[i];
    }
    if (SPLIT) {
      uint4* dl = reinterpret_cast<uint4*>(as_lo + lrow * kLdsStride + lk);
#pragma unroll
      for (int i = 0; i < 4; i++) dl[i] = ra_lo[i];
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.0f;

  const int fr = lane & 31;        // fragment row/column
  const int fk = (lane >> 5) * 8;  // fragment k offset within a 16-wide step
  const int nk = K / kBK;
  load_regs(0);
  for (int ks = 0; ks < nk; ks++) {
    __syncthreads();
    store_lds();
    __syncthreads();
    if (ks + 1 < nk) load_regs((ks + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 16) {
      bf16x8 a_hi[2], a_lo[2], b[2];
#pragma unroll
      for (int mi = 0; mi < 2; mi++) {
        const int row = wm * 64 + mi * 32 + fr;
        a_hi[mi] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(as_hi + row * kLdsStride + kk + fk));
        if (SPLIT)
          a_lo[mi] = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const uint4*>(as_lo + row * kLdsStride + kk + fk));
      }
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        const int col = wn * 64 + ni * 32 + fr;
        b[ni] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(bs + col * kLdsStride + kk + fk));
      }
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
          acc[mi][ni] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_hi[mi], b[ni], acc[mi][ni], 0, 0, 0);
          if (SPLIT)
            acc[mi][ni] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_lo[mi], b[ni], acc[mi][ni], 0, 0, 0);
        }
    }
  }

  // Output element (mi, ni, r) of this lane: row wm*64 + mi*32 +
  // 8*(r/4) + 4*(lane/32) + r%4, column wn*64 + ni*32 + lane%32.
  if (GATEUP) {
    const int col = (n0 + wn * 64) / 2 + fr;  // hidden column of this lane
    uint16_t* h_hi = routed ? P.h_hi : P.hs_hi;
    uint16_t* h_lo = routed ? P.h_lo : P.hs_lo;
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < mrows) {
          const float h = silu(acc[mi][0][r]) * acc[mi][1][r];
          const size_t at = (size_t)(base + r0 + row) * W + col;
          const uint16_t hb = bf16_bits(h);
          h_hi[at] = hb;
          if (SPLIT) h_lo[at] = bf16_bits(h - __uint_as_float((uint32_t)hb << 16));
        }
      }
  } else {
    float* out = routed ? S.y : S.ys;
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        const int col = n0 + wn * 64 + ni * 32 + fr;
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row < mrows) out[(size_t)(base + r0 + row) * L.H + col] = acc[mi][ni][r];
        }
      }
  }
}

void launch_split_planes(const float* x, size_t n, uint16_t* hi, uint16_t* lo, hipStream_t s) {
  if (n == 0) return;
  const size_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     s, x, n, hi, lo);
}

void launch_mfma_gateup(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, hipStream_t s) {
  dim3 grid((2 * L.S + kBN - 1) / kBN, tiles_bound);
  if (bf16_only)
    hipLaunchKernelGGL((mfma_group_kernel<false, true>), grid, dim3(256), 0, s, L, S, P, T);
  else
    hipLaunchKernelGGL((mfma_group_kernel<true, true>), grid, dim3(256), 0, s, L, S, P, T);
}

void launch_mfma_down(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                      int tiles_bound, bool bf16_only, hipStream_t s) {
  dim3 grid((L.H + kBN - 1) / kBN, tiles_bound);
  if (bf16_only)
    hipLaunchKernelGGL((mfma_group_kernel<false, false>), grid, dim3(256), 0, s, L, S, P, T);
  else
    hipLaunchKernelGGL((mfma_group_kernel<true, false>), grid, dim3(256), 0, s, L, S, P, T);
}

}  // namespace uocr
