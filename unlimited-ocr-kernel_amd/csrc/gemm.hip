// MFMA grouped GEMM engine for multi-token batches (prefill), BF16 weights.
//
// Reference roles: the per-expert GEMMs of Decoder::experts / feed_forward
// (src/decoder/mod.rs:114-122, 197-218), which the reference runs as
// widened-FP32 scalar GEMMs (src/cpu/ops.rs:39-47, 119-132).
//
// A workgroup of 8 waves computes a 256x256 output tile of one expert group
// with v_mfma_f32_32x32x16_bf16; wave (wm, wn) owns rows [128 wm, +128) and
// columns [64 wn, +64) as 4x2 MFMA tiles. K is walked in 32-deep stages that
// global->LDS loads (no register staging) bring into a ring of LDS buffers,
// several stages ahead of the one being multiplied; the two waves of each
// SIMD alternate between multiplying and memory work (ping-pong), one
// barrier-separated phase apart. Weights are exact in bf16. FP32
// activations enter as bf16 planes: FP32-class precision splits each value
// x = hi + lo (relative residual <= 2^-18) and multiplies both planes; BF16
// activations use hi.
//
// Gate/up rows are interleaved in blocks of 32 (gate j.., up j..), so the
// wave whose 64 columns are one (gate, up) block pair holds g and u for the
// same (row, column) in the same lane and register: SiLU(g) * u is
// register-local and h leaves as bf16 planes for the down GEMM.
//
// Work items are (row tile, column tile) pairs enumerated on the device.
// Workgroup ids reach the 8 XCDs round-robin; they are remapped so each XCD
// takes a contiguous, cost-balanced range of the existing items, keeping an
// expert's weights in that XCD's L2.
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kTileM = 256, kTileN = 256, kXcds = 8;

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

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Global -> LDS load that bypasses registers (buffer_load_dwordx4 ... lds):
// lane l's 16 bytes land at LDS address M0 + 16 l, M0 being the wave-uniform
// `lds_addr`. Range-checked like any raw buffer load: offsets at or past the
// resource size write zeros. Written as inline assembly so the compiler does
// not treat it as an LDS store to wait for before every LDS read; the
// kernel waits on vmcnt itself before the barrier that publishes a stage.
// M0 is reserved to the compiler, which uses it only for such LDS transfers
// (none of its own here), so the asm sets it without declaring it.
__device__ __forceinline__ void buffer_load_lds16(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory");
}

__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  i32x4 r;
  r.x = (int)(uint32_t)a;
  r.y = (int)((a >> 32) & 0xffffu);  // stride 0
  r.z = (int)bytes;
  r.w = 0x00020000;  // gfx9 raw buffer word 3
  return r;
}

constexpr uint32_t kDmaOut = 0x80000000u;  // offset past every resource

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt
// bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at maximum).
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// SPLITB: INT8-overlay weights as dequantised bf16 hi + lo planes (a third
// product term), y always f32; groups of one row are skipped when the
// overlay runs DynamicActivations (the batch engine's W8A8 path owns them).
template <int WAVES, int BK, int NBUF, bool SPLIT, bool GATEUP, bool SPLITB = false>
__global__ __launch_bounds__(WAVES * 64, 1) void mfma_group_kernel(DeviceLayer L, Scratch S,
                                                                   MfmaPlanes P, int T) {
  // Waves form a 2 x (WAVES/2) grid over the 256 x 256 tile; each owns 128
  // rows and kWc columns as 4 x kNi MFMA tiles.
  constexpr int kWn = WAVES / 2;
  constexpr int kWc = kTileN / kWn;
  constexpr int kNi = kWc / 32;
  extern __shared__ __align__(16) uint16_t lds[];  // [stage][A hi | B | A lo | B lo]
  __shared__ int arow[kTileM];

  // ---- work item. Workgroup ids reach the XCDs round-robin (id % 8). The
  // items are listed shared-expert first, then routed (each in row-tile,
  // column-tile order), and cut into 8 contiguous ranges of equal cost, one
  // per XCD: an item costs its K depth, so the deeper shared items of the
  // down GEMM do not pile up on one XCD, neighbouring items (same expert,
  // same rows) meet in one L2, and an XCD's deeper items start first.
  const int routed_tiles = S.counters[1];
  const int all_tiles = S.counters[0];
  const int n_routed = GATEUP ? 2 * L.I : L.H;
  const int n_shared = GATEUP ? 2 * L.S : L.H;
  const int nt_routed = (n_routed + kTileN - 1) / kTileN;
  const int nt_shared = (n_shared + kTileN - 1) / kTileN;
  const long long routed_items = (long long)routed_tiles * nt_routed;
  const long long shared_items = (long long)(all_tiles - routed_tiles) * nt_shared;
  const long long c_shared = GATEUP ? L.H : L.S, c_routed = GATEUP ? L.H : L.I;
  const long long shared_cost = shared_items * c_shared;
  const long long total_cost = shared_cost + routed_items * c_routed;
  // First item of XCD x: the first whose cost prefix reaches x / 8 of the total.
  auto first_item = [&](int x) -> long long {
    const long long b = total_cost * x / kXcds;
    if (b <= shared_cost) return (b + c_shared - 1) / c_shared;
    return shared_items + (b - shared_cost + c_routed - 1) / c_routed;
  };
  const int xcd = blockIdx.x % kXcds;
  const long long item = first_item(xcd) + blockIdx.x / kXcds;
  if (item >= first_item(xcd + 1)) return;
  int tile, ntile;
  if (item < shared_items) {
    tile = routed_tiles + (int)(item / nt_shared);
    ntile = (int)(item % nt_shared);
  } else {
    tile = (int)((item - shared_items) / nt_routed);
    ntile = (int)((item - shared_items) % nt_routed);
  }
  const int g = S.tiles[2 * tile], r0 = S.tiles[2 * tile + 1];
  const bool routed = g < L.E;
  const int W = L.width(g);
  const int N = GATEUP ? 2 * W : L.H;
  const int K = GATEUP ? L.H : W;
  const int n0 = ntile * kTileN;
  const int group_rows = routed ? S.offsets[g + 1] - S.offsets[g] : T;
  if (SPLITB && routed && group_rows == 1 && L.quant_mode == kQuantDynamic)
    return;
  const int mrows = min(kTileM, group_rows - r0);
  const int base = routed ? S.offsets[g] : 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / kWn, wn = wave % kWn;

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

  // ---- LDS tiles. A stage holds the A plane(s) and B, each [256 rows][BK]
  // bf16 with no padding: chunk c (8 bf16) of row r sits at position
  // c ^ swz(r), which spreads the 16-byte fragment reads of 16 consecutive
  // rows over all LDS banks. Loads arrive as 1 KB wave segments of
  // kSegRows rows (lane l -> row l / kCpr, position l % kCpr).
  constexpr int kCpr = BK / 8;                 // 16-byte chunks per row
  constexpr int kSegRows = 64 / kCpr;          // rows per 1 KB segment
  constexpr int kSegs = kTileM / kSegRows;     // segments per plane
  constexpr int kSegPerWave = kSegs / WAVES;   // per wave, per plane
  constexpr int kRowDiv = 16 / kCpr;
  auto swz = [](int r) { return (r / kRowDiv) % kCpr; };
  const uint32_t plane_bytes = (uint32_t)kTileM * BK * 2;
  constexpr int kPlanes = 2 + (SPLIT ? 1 : 0) + (SPLITB ? 1 : 0);
  const uint32_t stage_bytes = kPlanes * plane_bytes;
  const uint32_t blo_plane = (SPLIT ? 3 : 2) * plane_bytes;  // B lo, when SPLITB

  // Per-lane source offsets of this wave's segments (k = 0).
  const uint32_t row_bytes = (uint32_t)K * 2;
  uint32_t a_off[kSegPerWave], b_off[kSegPerWave];
#pragma unroll
  for (int i = 0; i < kSegPerWave; i++) {
    const int r = (wave * kSegPerWave + i) * kSegRows + lane / kCpr;
    const int c = (lane % kCpr) ^ swz(r);
    const int src_row = arow[r];
    a_off[i] = src_row >= 0 ? (uint32_t)src_row * row_bytes + 16u * c : kDmaOut;
    b_off[i] = n0 + r < N ? (uint32_t)(n0 + r) * row_bytes + 16u * c : kDmaOut;
  }
  const uint16_t* a_hi_src;
  const uint16_t* a_lo_src;
  uint32_t a_rows;
  if (GATEUP) {
    a_hi_src = P.x_hi;
    a_lo_src = P.x_lo;
    a_rows = (uint32_t)T;
  } else {
    a_hi_src = routed ? P.h_hi : P.hs_hi;
    a_lo_src = routed ? P.h_lo : P.hs_lo;
    a_rows = routed ? (uint32_t)T * L.K : (uint32_t)T;
  }
  const uint16_t* wmat;
  const uint16_t* wmat_lo = nullptr;
  if constexpr (SPLITB) {
    wmat = GATEUP ? L.dq13 + L.w13_offset(g) : L.dq2 + L.w2_offset(g);
    wmat_lo = wmat + (GATEUP ? L.n13() : L.n2());
  } else {
    wmat = GATEUP ? L.w13 + L.w13_offset(g) : L.w2 + L.w2_offset(g);
  }
  const i32x4 rs_a = buffer_rsrc(a_hi_src, a_rows * row_bytes);
  const i32x4 rs_l = buffer_rsrc(a_lo_src, a_rows * row_bytes);
  const i32x4 rs_b = buffer_rsrc(wmat, (uint32_t)N * row_bytes);
  const i32x4 rs_bl = buffer_rsrc(SPLITB ? wmat_lo : wmat, (uint32_t)N * row_bytes);
  // LDS byte address of this wave's first segment of stage buffer 0.
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)lds) +
      (uint32_t)wave * kSegPerWave * 1024u);
  auto issue = [&](int buf, int k0) {
    const uint32_t st = lds0 + (uint32_t)buf * stage_bytes;
    const uint32_t kb = (uint32_t)k0 * 2u;
#pragma unroll
    for (int i = 0; i < kSegPerWave; i++) {
      buffer_load_lds16(rs_a, st + i * 1024u, a_off[i] + kb);
      buffer_load_lds16(rs_b, st + plane_bytes + i * 1024u, b_off[i] + kb);
      if constexpr (SPLIT) buffer_load_lds16(rs_l, st + 2 * plane_bytes + i * 1024u, a_off[i] + kb);
      if constexpr (SPLITB) buffer_load_lds16(rs_bl, st + blo_plane + i * 1024u, b_off[i] + kb);
    }
  };

  floatx16 acc[4][kNi];
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < kNi; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.0f;

  const int fr = lane & 31;   // fragment row / column
  const int fc = lane >> 5;   // fragment chunk inside a 16-wide k step
  const int nk = K / BK;

  // Ping-pong schedule. The two waves sharing a SIMD (w and w + 4) are in
  // opposite groups, one phase apart: while one group multiplies stage ks
  // from registers, the other reads its stage-ks fragments from LDS and
  // issues the global loads of stage ks + kDepth, so each SIMD's MFMA pipe
  // is fed by one wave while its partner does memory work. Every phase ends
  // at a workgroup barrier (group 1 passes one extra at the start, group 0
  // one at the end, so both pass 2 nk + 1).
  //
  // Buffers: stage s lives in buffer s % NBUF, NBUF = kDepth + 1. The loads
  // of stage ks + kDepth overwrite stage ks - 1, whose last reader (group 1,
  // the phase before) finished its reads before that phase's barrier. Each
  // wave issues kLps loads per stage, and vmcnt retires them in order, so at
  // the end of a memory phase "own loads of stage ks + 1 landed" is
  // vmcnt <= (kDepth - 1) * kLps; the barrier then publishes them to both
  // groups before either reads stage ks + 1.
  static_assert(WAVES == 8, "the ping-pong schedule pairs two waves per SIMD");
  constexpr int kDepth = NBUF - 1;
  constexpr int kLps = kSegPerWave * kPlanes;
  constexpr int kSub = BK / 16;
  const int grp = wave >> 2;
  for (int i = 0; i < kDepth; i++)
    if (i < nk) issue(i, i * BK);
  if (nk >= kDepth)
    __builtin_amdgcn_s_waitcnt(vmcnt_only((kDepth - 1) * kLps));
  else
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
  __syncthreads();
  if (grp) __syncthreads();
  for (int ks = 0; ks < nk; ks++) {
    // ---- memory phase
    const bool steady = ks + kDepth < nk;
    if (steady) issue((ks + kDepth) % NBUF, (ks + kDepth) * BK);
    const char* cur = reinterpret_cast<const char*>(lds) + (ks % NBUF) * stage_bytes;
    bf16x8 fa[kSub][4], fl[kSub][SPLIT ? 4 : 1], fb[kSub][kNi], fbl[kSub][SPLITB ? kNi : 1];
    auto frag = [&](const char* plane, int row, int c) {
      return as_bf16x8(*reinterpret_cast<const uint4*>(plane + row * (BK * 2) + 16 * (c ^ swz(row))));
    };
#pragma unroll
    for (int sub = 0; sub < kSub; sub++) {
      const int c = 2 * sub + fc;
#pragma unroll
      for (int ni = 0; ni < kNi; ni++) {
        fb[sub][ni] = frag(cur + plane_bytes, wn * kWc + ni * 32 + fr, c);
        if constexpr (SPLITB) fbl[sub][ni] = frag(cur + blo_plane, wn * kWc + ni * 32 + fr, c);
      }
#pragma unroll
      for (int mi = 0; mi < 4; mi++) {
        fa[sub][mi] = frag(cur, wm * 128 + mi * 32 + fr, c);
        if constexpr (SPLIT) fl[sub][mi] = frag(cur + 2 * plane_bytes, wm * 128 + mi * 32 + fr, c);
      }
    }
    if (steady)
      __builtin_amdgcn_s_waitcnt(vmcnt_only((kDepth - 1) * kLps));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    // ---- compute phase. Gate/up puts the weight fragment first, so each
    // accumulator holds a [32 features x 32 tokens] block (lane l owns token
    // l % 32 and four consecutive features per register quad: h leaves in
    // 8-byte stores). Down keeps [32 tokens x 32 features] (lane l owns
    // feature l % 32: a half-wave writes 32 adjacent outputs of one row).
    auto mma = [&](const bf16x8& a, const bf16x8& b, floatx16& c) {
      c = GATEUP ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0)
                 : __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    };
#pragma unroll
    for (int sub = 0; sub < kSub; sub++)
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < kNi; ni++) {
          mma(fa[sub][mi], fb[sub][ni], acc[mi][ni]);
          if constexpr (SPLIT) mma(fl[sub][mi], fb[sub][ni], acc[mi][ni]);
          if constexpr (SPLITB) mma(fa[sub][mi], fbl[sub][ni], acc[mi][ni]);
        }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  }
  if (!grp) __syncthreads();

  const int wcol0 = n0 + wn * kWc;
  if (wcol0 >= N) return;
  if (GATEUP) {
    // Output element (mi, ni, r) of this lane: token row 128 wm + 32 mi +
    // lane%32, feature column kWc wn + 32 ni + 8 (r/4) + 4 (lane/32) + r%4;
    // registers 4j .. 4j+3 are four consecutive features of one token.
    // Columns 64b .. 64b+63 of the wave are one (gate, up) block pair.
    // SiLU(g) u = g / (1 + exp(-g)) u with a hardware reciprocal.
    uint16_t* h_hi = routed ? P.h_hi : P.hs_hi;
    uint16_t* h_lo = routed ? P.h_lo : P.hs_lo;
#pragma unroll
    for (int bp = 0; bp < kNi / 2; bp++) {
      if (wcol0 + 64 * bp >= N) break;
      const int col0 = (wcol0 + 64 * bp) / 2 + 4 * fc;  // hidden column of register 0
#pragma unroll
      for (int mi = 0; mi < 4; mi++) {
        const int row = wm * 128 + 32 * mi + fr;
        if (row >= mrows) continue;
        const size_t at0 = (size_t)(base + r0 + row) * W + col0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          uint32_t hb[4], lb[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float gv = acc[mi][2 * bp][4 * j + i];
            const float h = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * acc[mi][2 * bp + 1][4 * j + i];
            hb[i] = bf16_bits(h);
            if constexpr (SPLIT) lb[i] = bf16_bits(h - __uint_as_float(hb[i] << 16));
          }
          *reinterpret_cast<uint2*>(h_hi + at0 + 8 * j) =
              make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
          if constexpr (SPLIT)
            *reinterpret_cast<uint2*>(h_lo + at0 + 8 * j) =
                make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16));
        }
      }
    }
  } else {
    // Output element (mi, ni, r) of this lane: row 128 wm + 32 mi + 8 (r/4)
    // + 4 (lane/32) + r%4, column kWc wn + 32 ni + lane%32.
    // FP32-class and INT8 weights: y in f32. BF16 weights with BF16
    // activations: y rounded to bf16 (the combine's operands), in the first
    // half of the same buffer.
    float* out = routed ? S.y : S.ys;
    uint16_t* out16 = reinterpret_cast<uint16_t*>(out);
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < kNi; ni++) {
        const int col = wcol0 + ni * 32 + fr;
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = wm * 128 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row >= mrows) continue;
          const size_t at = (size_t)(base + r0 + row) * L.H + col;
          if constexpr (SPLIT || SPLITB)
            out[at] = acc[mi][ni][r];
          else
            out16[at] = bf16_bits(acc[mi][ni][r]);
        }
      }
  }
}

template <int BK, int NBUF, int PLANES>
constexpr size_t mfma_lds_bytes() {
  return (size_t)NBUF * PLANES * kTileM * BK * sizeof(uint16_t);
}
// BF16 activations: 32-deep stages, four buffers (128 KiB). FP32-class
// (hi + lo planes): 32-deep stages, three buffers (144 KiB). INT8 overlay
// (dequantised weight hi + lo planes, and the activation's lo plane in the
// FP32 class): 16-deep stages, four buffers (96 / 128 KiB).
constexpr int kBkBf16 = 32, kBufBf16 = 4, kBkSplit = 32, kBufSplit = 3;
constexpr int kBkQ = 16, kBufQ = 4;
constexpr int kWaves = 8;

// INT8 overlay -> bf16 planes of the dequantised weight: w = q * s rounded to
// f32 as Int8Matrix::linear does (src/cpu/quantized.rs:119-131), then hi =
// bf16(w) and lo = bf16(w - hi) (|w - hi - lo| <= 2^-16 |w|). Row-major
// [rows, cols] with scales [rows, cols / 32].
__global__ void dequant_planes_kernel(const int8_t* __restrict__ q, const float* __restrict__ sc,
                                      size_t n, int cols, uint16_t* __restrict__ hi,
                                      uint16_t* __restrict__ lo) {
  for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < n;
       i += (size_t)gridDim.x * blockDim.x * 4) {
    const char4 v = *reinterpret_cast<const char4*>(q + i);
    const int8_t qv[4] = {v.x, v.y, v.z, v.w};
    uint16_t h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const size_t e = i + j;
      const float w = (float)qv[j] * sc[(e / cols) * (cols / 32) + (e % cols) / 32];
      h[j] = bf16_bits(w);
      l[j] = bf16_bits(w - __uint_as_float((uint32_t)h[j] << 16));
    }
    *reinterpret_cast<uint2*>(hi + i) =
        make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
    *reinterpret_cast<uint2*>(lo + i) =
        make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
  }
}

void launch_dequant_planes(const int8_t* q, const float* sc, size_t n, int cols, uint16_t* hi,
                           uint16_t* lo, hipStream_t s) {
  if (n == 0) return;
  hipLaunchKernelGGL(dequant_planes_kernel, dim3(4096), dim3(256), 0, s, q, sc, n, cols, hi, lo);
}

void launch_split_planes(const float* x, size_t n, uint16_t* hi, uint16_t* lo, hipStream_t s) {
  if (n == 0) return;
  const size_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     s, x, n, hi, lo);
}

// Workgroups: 8 XCDs times the most items one XCD can take. Items are
// bounded by every row tile times the widest column count; an XCD's range
// holds an eighth of the cost, so at most (bound / 8) * (deepest / shallowest
// item) + 2 items.
static unsigned mfma_grid(const DeviceLayer& L, int tiles_bound, bool gateup) {
  const int n = gateup ? std::max(2 * L.S, 2 * L.I) : L.H;
  const long long items = (long long)tiles_bound * ((n + kTileN - 1) / kTileN);
  const long long deep = gateup ? 1 : std::max(L.S, L.I), shallow = gateup ? 1 : std::min(L.S, L.I);
  const long long per_xcd = (items * deep + kXcds * shallow - 1) / (kXcds * shallow) + 2;
  return (unsigned)(per_xcd * kXcds);
}

template <bool GATEUP>
static void launch_mfma(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, hipStream_t s) {
  const dim3 grid(mfma_grid(L, tiles_bound, GATEUP)), block(kWaves * 64);
  if (L.quant_mode != kQuantNone) {
    if (bf16_only)
      mfma_group_kernel<kWaves, kBkQ, kBufQ, false, GATEUP, true>
          <<<grid, block, mfma_lds_bytes<kBkQ, kBufQ, 3>(), s>>>(L, S, P, T);
    else
      mfma_group_kernel<kWaves, kBkQ, kBufQ, true, GATEUP, true>
          <<<grid, block, mfma_lds_bytes<kBkQ, kBufQ, 4>(), s>>>(L, S, P, T);
  } else if (bf16_only) {
    mfma_group_kernel<kWaves, kBkBf16, kBufBf16, false, GATEUP>
        <<<grid, block, mfma_lds_bytes<kBkBf16, kBufBf16, 2>(), s>>>(L, S, P, T);
  } else {
    mfma_group_kernel<kWaves, kBkSplit, kBufSplit, true, GATEUP>
        <<<grid, block, mfma_lds_bytes<kBkSplit, kBufSplit, 3>(), s>>>(L, S, P, T);
  }
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
  auto set = [](const void* k, size_t bytes) {
    (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  };
  set((const void*)mfma_group_kernel<kWaves, kBkBf16, kBufBf16, false, true>,
      mfma_lds_bytes<kBkBf16, kBufBf16, 2>());
  set((const void*)mfma_group_kernel<kWaves, kBkBf16, kBufBf16, false, false>,
      mfma_lds_bytes<kBkBf16, kBufBf16, 2>());
  set((const void*)mfma_group_kernel<kWaves, kBkSplit, kBufSplit, true, true>,
      mfma_lds_bytes<kBkSplit, kBufSplit, 3>());
  set((const void*)mfma_group_kernel<kWaves, kBkSplit, kBufSplit, true, false>,
      mfma_lds_bytes<kBkSplit, kBufSplit, 3>());
  set((const void*)mfma_group_kernel<kWaves, kBkQ, kBufQ, false, true, true>,
      mfma_lds_bytes<kBkQ, kBufQ, 3>());
  set((const void*)mfma_group_kernel<kWaves, kBkQ, kBufQ, false, false, true>,
      mfma_lds_bytes<kBkQ, kBufQ, 3>());
  set((const void*)mfma_group_kernel<kWaves, kBkQ, kBufQ, true, true, true>,
      mfma_lds_bytes<kBkQ, kBufQ, 4>());
  set((const void*)mfma_group_kernel<kWaves, kBkQ, kBufQ, true, false, true>,
      mfma_lds_bytes<kBkQ, kBufQ, 4>());
  (void)hipGetLastError();  // a refused attribute surfaces at launch instead
}

}  // namespace uocr
