// MFMA grouped GEMM engine for multi-token batches (prefill), BF16 weights.
//
// Reference roles: the per-expert GEMMs of Decoder::experts / feed_forward
// (src/decoder/mod.rs:114-122, 197-218), which the reference runs as
// widened-FP32 scalar GEMMs (src/cpu/ops.rs:39-47, 119-132).
//
// A workgroup of 8 waves computes a 256x256 output tile of one expert group
// with v_mfma_f32_32x32x16_bf16; wave (wm, wn) owns rows [128 wm, +128) and
// columns [64 wn, +64) as 4x2 MFMA tiles whose accumulators live in AGPRs.
// K is walked in stages staged through double-buffered LDS (rows padded by
// 16 bytes, which keeps 128-bit LDS reads and writes free of bank
// conflicts); the global loads of stage k+2 are in flight while stage k is
// multiplied. Weights are exact in bf16. FP32 activations enter as bf16
// planes: FP32-class precision splits each value x = hi + lo (relative
// residual <= 2^-18) and multiplies both planes; BF16 activations use hi.
//
// Gate/up rows are interleaved in blocks of 32 (gate j.., up j..), so the
// wave whose 64 columns are one (gate, up) block pair holds g and u for the
// same (row, column) in the same lane and register: SiLU(g) * u is
// register-local and h leaves as bf16 planes for the down GEMM.
//
// Work items are (row tile, column tile) pairs enumerated on the device.
// Workgroup ids reach the 8 XCDs round-robin; they are remapped so each XCD
// takes a contiguous range of the existing items, keeping an expert's
// weights in that XCD's L2.
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kTileM = 256, kTileN = 256, kThreads = 512, kXcds = 8;

__device__ __forceinline__ uint16_t bf16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (__bf16)v);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

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

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;

// 16-byte load from global memory (explicit address space: the compiler
// then issues global loads whose completion it can wait for lazily).
__device__ __forceinline__ u32x4 gload16(const uint16_t* p) { return *(global_u32x4*)(p); }

// Rows past the tile's valid range load row 0 of the same matrix instead
// (always in bounds): an MFMA output row depends only on its own A row and
// an output column only on its own B row, and those rows and columns are
// never written back, so no select is needed and the loads stay in flight.
template <int KV>
__device__ __forceinline__ void load_stage(u32x4 (&dst)[KV], const uint16_t* p) {
#pragma unroll
  for (int i = 0; i < KV; i++) dst[i] = gload16(p + 8 * i);
}

template <int KV>
__device__ __forceinline__ void store_stage(uint16_t* dst, const u32x4 (&src)[KV]) {
#pragma unroll
  for (int i = 0; i < KV; i++) *reinterpret_cast<u32x4*>(dst + 8 * i) = src[i];
}

template <int BK, bool SPLIT, bool GATEUP>
__global__ __launch_bounds__(kThreads, 1) void mfma_group_kernel(DeviceLayer L, Scratch S,
                                                                 MfmaPlanes P, int T) {
  constexpr int kStride = BK + 8;              // bf16 per LDS row
  constexpr int kPlane = kTileM * kStride;     // bf16 per plane per stage
  constexpr int kVec = BK / 16;
  extern __shared__ __align__(16) uint16_t lds[];
  // Layout: [stage][A hi | B | A lo] planes.
  uint16_t* const stage0 = lds;
  uint16_t* const stage1 = lds + (SPLIT ? 3 : 2) * kPlane;
  __shared__ int arow[kTileM];

  // ---- work item. Workgroup ids reach the XCDs round-robin (id % 8); XCD
  // x takes the contiguous item range [x * chunk, (x + 1) * chunk) of the
  // items that exist, so all 8 XCDs share the work and neighbouring items
  // (same expert) meet in one L2.
  const int routed_tiles = S.counters[1];
  const int all_tiles = S.counters[0];
  const int n_routed = GATEUP ? 2 * L.I : L.H;
  const int n_shared = GATEUP ? 2 * L.S : L.H;
  const int nt_routed = (n_routed + kTileN - 1) / kTileN;
  const int nt_shared = (n_shared + kTileN - 1) / kTileN;
  const int routed_items = routed_tiles * nt_routed;
  const int n_items = routed_items + (all_tiles - routed_tiles) * nt_shared;
  const int chunk = (n_items + kXcds - 1) / kXcds;
  const int slot = blockIdx.x / kXcds;
  const int item = (blockIdx.x % kXcds) * chunk + slot;
  if (slot >= chunk || item >= n_items) return;
  int tile, ntile;
  if (item < routed_items) {
    tile = item / nt_routed;
    ntile = item % nt_routed;
  } else {
    const int rest = item - routed_items;
    tile = routed_tiles + rest / nt_shared;
    ntile = rest % nt_shared;
  }
  const int g = S.tiles[2 * tile], r0 = S.tiles[2 * tile + 1];
  const bool routed = g < L.E;
  const int W = L.width(g);
  const int N = GATEUP ? 2 * W : L.H;
  const int K = GATEUP ? L.H : W;
  const int n0 = ntile * kTileN;
  const int group_rows = routed ? S.offsets[g + 1] - S.offsets[g] : T;
  const int mrows = min(kTileM, group_rows - r0);
  const int base = routed ? S.offsets[g] : 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  if (tid < kTileM) {
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

  // Thread -> (row, k part) for global loads: two threads per row.
  const int lrow = tid >> 1;
  const int lk = (tid & 1) * (BK / 2);
  const int src_row = arow[lrow];
  const bool a_ok = src_row >= 0;
  const bool b_ok = n0 + lrow < N;
  const uint16_t* a_hi_ptr = a_hi_src + (size_t)(a_ok ? src_row : 0) * K + lk;
  const uint16_t* a_lo_ptr = a_lo_src + (size_t)(a_ok ? src_row : 0) * K + lk;
  const uint16_t* b_ptr = wmat + (size_t)(b_ok ? n0 + lrow : 0) * K + lk;

  u32x4 ra[kVec], rl[SPLIT ? kVec : 1], rb[kVec];
  floatx16 acc[4][2];
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.0f;

  const int fr = lane & 31;        // fragment row / column
  const int fk = (lane >> 5) * 8;  // fragment k offset inside a 16-wide step
  const int nk = K / BK;

  const int a_off = lrow * kStride + lk;
  auto issue = [&](int k0) {
    load_stage<kVec>(ra, a_hi_ptr + k0);
    load_stage<kVec>(rb, b_ptr + k0);
    if constexpr (SPLIT) load_stage<kVec>(rl, a_lo_ptr + k0);
  };
  auto commit = [&](uint16_t* st) {
    store_stage<kVec>(st + a_off, ra);
    store_stage<kVec>(st + kPlane + a_off, rb);
    if constexpr (SPLIT) store_stage<kVec>(st + 2 * kPlane + a_off, rl);
  };
  issue(0);
  commit(stage0);
  if (nk > 1) issue(BK);
  __syncthreads();
  for (int ks = 0; ks < nk; ks++) {
    const uint16_t* cur = (ks & 1) ? stage1 : stage0;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a[4], al[4], b[2];
#pragma unroll
      for (int mi = 0; mi < 4; mi++) {
        const int row = wm * 128 + mi * 32 + fr;
        a[mi] = as_bf16x8(*reinterpret_cast<const uint4*>(cur + row * kStride + kk + fk));
        if constexpr (SPLIT)
          al[mi] = as_bf16x8(
              *reinterpret_cast<const uint4*>(cur + 2 * kPlane + row * kStride + kk + fk));
      }
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        const int col = wn * 64 + ni * 32 + fr;
        b[ni] = as_bf16x8(*reinterpret_cast<const uint4*>(cur + kPlane + col * kStride + kk + fk));
      }
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
          if constexpr (SPLIT)
            acc[mi][ni] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[mi], b[ni], acc[mi][ni], 0, 0, 0);
        }
    }
    if (ks + 1 < nk) {
      commit((ks & 1) ? stage0 : stage1);
      if (ks + 2 < nk) issue((ks + 2) * BK);
    }
    __syncthreads();
  }

  // Output element (mi, ni, r) of this lane: row 128 wm + 32 mi + 8 (r/4) +
  // 4 (lane/32) + r%4, column 64 wn + 32 ni + lane%32.
  const int wcol0 = n0 + wn * 64;
  if (wcol0 >= N) return;
  if (GATEUP) {
    const int col = wcol0 / 2 + fr;  // hidden column of this lane
    uint16_t* h_hi = routed ? P.h_hi : P.hs_hi;
    uint16_t* h_lo = routed ? P.h_lo : P.hs_lo;
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = wm * 128 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < mrows) {
          const float gv = acc[mi][0][r];
          const float h = __fdividef(gv, 1.0f + __expf(-gv)) * acc[mi][1][r];
          const size_t at = (size_t)(base + r0 + row) * W + col;
          const uint16_t hb = bf16_bits(h);
          h_hi[at] = hb;
          if constexpr (SPLIT) h_lo[at] = bf16_bits(h - __uint_as_float((uint32_t)hb << 16));
        }
      }
  } else {
    float* out = routed ? S.y : S.ys;
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        const int col = wcol0 + ni * 32 + fr;
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = wm * 128 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row < mrows) out[(size_t)(base + r0 + row) * L.H + col] = acc[mi][ni][r];
        }
      }
  }
}

template <int BK, bool SPLIT>
constexpr size_t mfma_lds_bytes() {
  return (size_t)2 * (SPLIT ? 3 : 2) * kTileM * (BK + 8) * sizeof(uint16_t);
}

void launch_split_planes(const float* x, size_t n, uint16_t* hi, uint16_t* lo, hipStream_t s) {
  if (n == 0) return;
  const size_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     s, x, n, hi, lo);
}

// Upper bound of work items: every row tile times the widest column count,
// rounded up to a multiple of the XCD count.
static unsigned mfma_grid(const DeviceLayer& L, int tiles_bound, bool gateup) {
  const int n = gateup ? 2 * L.S : L.H;
  const long long items = (long long)tiles_bound * ((n + kTileN - 1) / kTileN);
  return (unsigned)((items + kXcds - 1) / kXcds * kXcds);
}

template <bool GATEUP>
static void launch_mfma(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, hipStream_t s) {
  const dim3 grid(mfma_grid(L, tiles_bound, GATEUP));
  if (bf16_only)
    mfma_group_kernel<64, false, GATEUP>
        <<<grid, dim3(kThreads), mfma_lds_bytes<64, false>(), s>>>(L, S, P, T);
  else
    mfma_group_kernel<32, true, GATEUP>
        <<<grid, dim3(kThreads), mfma_lds_bytes<32, true>(), s>>>(L, S, P, T);
}

void launch_mfma_gateup(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, hipStream_t s) {
  launch_mfma<true>(L, S, P, T, tiles_bound, bf16_only, s);
}

void launch_mfma_down(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                      int tiles_bound, bool bf16_only, hipStream_t s) {
  launch_mfma<false>(L, S, P, T, tiles_bound, bf16_only, s);
}

void mfma_init_attributes() {
  (void)hipFuncSetAttribute((const void*)mfma_group_kernel<64, false, true>,
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)mfma_lds_bytes<64, false>());
  (void)hipFuncSetAttribute((const void*)mfma_group_kernel<64, false, false>,
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)mfma_lds_bytes<64, false>());
  (void)hipFuncSetAttribute((const void*)mfma_group_kernel<32, true, true>,
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)mfma_lds_bytes<32, true>());
  (void)hipFuncSetAttribute((const void*)mfma_group_kernel<32, true, false>,
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)mfma_lds_bytes<32, true>());
  (void)hipGetLastError();  // a refused attribute surfaces at launch instead
}

}  // namespace uocr
