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
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
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

// Global -> LDS load of one dword per lane (lane l -> M0 + 4 l).
__device__ __forceinline__ void buffer_load_lds4(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory");
}

// Scalar read of a dword this kernel never writes (the dispatch tables),
// waited for on the spot. Written as assembly so the read stays on the
// scalar path inside a loop that also stores, where the compiler would
// otherwise read through the vector path and wait on vmcnt, which the
// global -> LDS pipeline keeps busy.
__device__ __forceinline__ int scalar_read(const int* p) {
  // The address is workgroup-uniform; readfirstlane puts it in SGPRs.
  const unsigned long long a = reinterpret_cast<unsigned long long>(p);
  const unsigned long long u =
      (unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a) |
      ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32);
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(u) : "memory");
  return __builtin_amdgcn_readfirstlane(v);  // tells the compiler the value is uniform
}

// One work item: a (row tile, column tile) of one expert group. Every
// field is workgroup-uniform.
struct MfmaItem {
  int g, r0, base, mrows, W, N, K, n0, nk;
  bool routed;
};

template <int WAVES, int BK, int NBUF, bool SPLIT, bool GATEUP>
__global__ __launch_bounds__(WAVES * 64, 1) void mfma_group_kernel(DeviceLayer L, Scratch S,
                                                                   MfmaPlanes P, int T) {
  // Waves form a 2 x (WAVES/2) grid over the 256 x 256 tile; each owns 128
  // rows and kWc columns as 4 x kNi MFMA tiles.
  constexpr int kWn = WAVES / 2;
  constexpr int kWc = kTileN / kWn;
  constexpr int kNi = kWc / 32;
  extern __shared__ __align__(16) uint16_t lds[];  // [NBUF][A hi | B | A lo], then arow[2][256]

  // ---- work items. Workgroup ids reach the XCDs round-robin (id % 8). The
  // items are listed shared-expert first, then routed (each in row-tile,
  // column-tile order), and cut into 8 contiguous ranges of equal cost, one
  // per XCD: an item costs its K depth, so the deeper shared items of the
  // down GEMM do not pile up on one XCD, and neighbouring items (same
  // expert, same rows) meet in one L2. The workgroup is persistent: it
  // takes every per-th item of its XCD's range (per = workgroups per XCD),
  // and its global -> LDS load stream runs on across item boundaries.
  const int routed_tiles = S.counters[1];
  const int all_tiles = S.counters[0];
  const int nt_routed = ((GATEUP ? 2 * L.I : L.H) + kTileN - 1) / kTileN;
  const int nt_shared = ((GATEUP ? 2 * L.S : L.H) + kTileN - 1) / kTileN;
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
  const int per = gridDim.x / kXcds;
  const long long lo = first_item(xcd) + blockIdx.x / kXcds, hi = first_item(xcd + 1);
  if (lo >= hi) return;
  const int n_my = (int)((hi - lo + per - 1) / per);
  auto describe = [&](int k) {
    const long long item = lo + (long long)k * per;
    int tile, ntile;
    if (item < shared_items) {
      tile = routed_tiles + (int)(item / nt_shared);
      ntile = (int)(item % nt_shared);
    } else {
      tile = (int)((item - shared_items) / nt_routed);
      ntile = (int)((item - shared_items) % nt_routed);
    }
    MfmaItem it;
    it.g = scalar_read(S.tiles + 2 * tile);
    it.r0 = scalar_read(S.tiles + 2 * tile + 1);
    it.routed = it.g < L.E;
    it.W = L.width(it.g);
    it.N = GATEUP ? 2 * it.W : L.H;
    it.K = GATEUP ? L.H : it.W;
    it.n0 = ntile * kTileN;
    it.base = it.routed ? scalar_read(S.offsets + it.g) : 0;
    const int group_rows = it.routed ? scalar_read(S.offsets + it.g + 1) - it.base : T;
    it.mrows = min(kTileM, group_rows - it.r0);
    it.nk = it.K / BK;
    return it;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / kWn, wn = wave % kWn;
  const int grp = wave >> 2;

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
  constexpr uint32_t plane_bytes = (uint32_t)kTileM * BK * 2;
  constexpr uint32_t stage_bytes = (SPLIT ? 3 : 2) * plane_bytes;
  const uint32_t lds_base =
      (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)lds);
  // Source rows of the gathered A tile (routed gate/up): arow[k & 1] holds
  // item k's, loaded by global -> LDS transfer one item ahead.
  int* arow = reinterpret_cast<int*>(reinterpret_cast<char*>(lds) + NBUF * stage_bytes);
  const uint32_t arow_lds = lds_base + NBUF * stage_bytes;
  auto load_arow = [&](const MfmaItem& it, int k) {
    if (!GATEUP || !it.routed || grp != 0) return;
    const i32x4 rs = buffer_rsrc(S.perm_rows + it.base + it.r0, (uint32_t)it.mrows * 4u);
    buffer_load_lds4(rs, __builtin_amdgcn_readfirstlane(arow_lds + (k & 1) * 1024u + wave * 256u),
                     (uint32_t)(wave * 64 + lane) * 4u);
  };

  // ---- the issue cursor: item ki, its stage si, global stage gi; the
  // resources and per-lane source offsets (k = 0) of its item.
  constexpr int kDepth = NBUF - 1;
  constexpr int kLps = kSegPerWave * (SPLIT ? 3 : 2);
  constexpr int kSps = BK / 32;  // 32-deep slices (ping-pong phases) per stage
  // An item spans at least kDepth stages (K >= 64): the issue cursor is at
  // most one item ahead, and item k + 1's source rows have landed (loads
  // older than a stage already waited for) when the cursor enters it.
  static_assert(kDepth * BK <= 64, "items must span at least kDepth stages");
  int ki = 0, si = 0, gi = 0;
  MfmaItem ii = describe(0);
  i32x4 rs_a, rs_l, rs_b;
  uint32_t a_off[kSegPerWave], b_off[kSegPerWave];
  auto enter_issue = [&](int k) {
    const uint32_t row_bytes = (uint32_t)ii.K * 2;
#pragma unroll
    for (int i = 0; i < kSegPerWave; i++) {
      const int r = (wave * kSegPerWave + i) * kSegRows + lane / kCpr;
      const int c = (lane % kCpr) ^ swz(r);
      int src = -1;
      if (r < ii.mrows) {
        if (GATEUP)
          src = ii.routed ? arow[(k & 1) * 256 + r] : ii.r0 + r;
        else
          src = ii.base + ii.r0 + r;
      }
      a_off[i] = src >= 0 ? (uint32_t)src * row_bytes + 16u * c : kDmaOut;
      b_off[i] = ii.n0 + r < ii.N ? (uint32_t)(ii.n0 + r) * row_bytes + 16u * c : kDmaOut;
    }
    const uint16_t* a_hi_src;
    const uint16_t* a_lo_src;
    uint32_t a_rows;
    if (GATEUP) {
      a_hi_src = P.x_hi;
      a_lo_src = P.x_lo;
      a_rows = (uint32_t)T;
    } else {
      a_hi_src = ii.routed ? P.h_hi : P.hs_hi;
      a_lo_src = ii.routed ? P.h_lo : P.hs_lo;
      a_rows = ii.routed ? (uint32_t)T * L.K : (uint32_t)T;
    }
    const uint16_t* wmat = GATEUP ? L.w13 + L.w13_offset(ii.g) : L.w2 + L.w2_offset(ii.g);
    rs_a = buffer_rsrc(a_hi_src, a_rows * row_bytes);
    rs_l = buffer_rsrc(a_lo_src, a_rows * row_bytes);
    rs_b = buffer_rsrc(wmat, (uint32_t)ii.N * row_bytes);
  };
  // LDS byte address of this wave's first segment of stage buffer 0.
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_base + (uint32_t)wave * kSegPerWave * 1024u);
  // Issue the next stage of the load stream (if any) into its ring buffer.
  auto issue_next = [&]() {
    if (ki >= n_my) return;
    const uint32_t st = lds0 + (uint32_t)(gi % NBUF) * stage_bytes;
    const uint32_t kb = (uint32_t)si * BK * 2u;
#pragma unroll
    for (int i = 0; i < kSegPerWave; i++) {
      buffer_load_lds16(rs_a, st + i * 1024u, a_off[i] + kb);
      buffer_load_lds16(rs_b, st + plane_bytes + i * 1024u, b_off[i] + kb);
      if constexpr (SPLIT) buffer_load_lds16(rs_l, st + 2 * plane_bytes + i * 1024u, a_off[i] + kb);
    }
    gi++;
    if (++si == ii.nk) {
      si = 0;
      if (++ki < n_my) {
        ii = describe(ki);
        enter_issue(ki);
        if (ki + 1 < n_my) load_arow(describe(ki + 1), ki + 1);
      }
    }
  };

  // ---- prologue: source rows of items 0 and 1, then kDepth stages.
  load_arow(ii, 0);
  if (n_my > 1) load_arow(describe(1), 1);
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
  __syncthreads();
  enter_issue(0);
  // Every wave has read item 0's rows before the stream may reuse arow[0].
  __syncthreads();
  for (int i = 0; i < kDepth; i++) issue_next();
  __builtin_amdgcn_s_waitcnt(vmcnt_only((kDepth - 1) * kLps));
  __syncthreads();

  floatx16 acc[4][kNi];
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < kNi; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.0f;

  const int fr = lane & 31;   // fragment row / column
  const int fc = lane >> 5;   // fragment chunk inside a 16-wide k step

  // ---- the compute cursor: item kc, its stage sc, global stage gc.
  //
  // Ping-pong schedule over 32-deep k slices (kSps per stage). The two
  // waves sharing a SIMD (w and w + 4) are in opposite groups, one phase
  // apart: while one group multiplies a slice from registers, the other
  // reads its fragments of the next slice from LDS (and, on a stage's first
  // slice, issues the next stage of the load stream), so each SIMD's MFMA
  // pipe is fed by one wave while its partner does memory work. Every phase
  // ends at a workgroup barrier (group 1 passes one extra at the start,
  // group 0 one at the end, so both pass the same number).
  //
  // Buffers: global stage s lives in buffer s % NBUF, NBUF = kDepth + 1.
  // The loads issued on stage gc's first slice (global stage gc + kDepth)
  // overwrite stage gc - 1, whose last reader (group 1, the phase before)
  // finished its reads before that phase's barrier. Each wave issues kLps
  // stage loads per stage (plus, in group 0, source-row loads, which only
  // make the waits below wait longer), and loads retire in order, so at the
  // end of a stage's last memory phase "own loads of stage gc + 1 landed" is
  // vmcnt <= (kDepth - 1) * kLps while the stream runs; the barrier then
  // publishes them to both groups before either reads stage gc + 1.
  static_assert(WAVES == 8, "the ping-pong schedule pairs two waves per SIMD");
  int kc = 0, sc = 0, gc = 0;
  MfmaItem ci = ii;
  // A tile with at most 128 real rows (a group's last) spreads them over
  // both wave rows: wave row wm owns rows [64 wm, +64) as 2 blocks instead
  // of [128 wm, +128) as 4. Blocks past the real rows are neither read
  // from LDS, multiplied nor stored.
  bool half = ci.mrows <= 128;
  int rbase = half ? wm * 64 : wm * 128;
  int live = __builtin_amdgcn_readfirstlane(min(half ? 2 : 4, max(0, (ci.mrows - rbase + 31) / 32)));
  if (grp) __syncthreads();
  for (;;) {
    const char* cur = reinterpret_cast<const char*>(lds) + (gc % NBUF) * stage_bytes;
#pragma unroll
    for (int sl = 0; sl < kSps; sl++) {
      // ---- memory phase: slice sl of global stage gc
      if (sl == 0) issue_next();
      bf16x8 fa[2][4], fl[2][SPLIT ? 4 : 1], fb[2][kNi];
      auto frag = [&](const char* plane, int row, int c) {
        return as_bf16x8(
            *reinterpret_cast<const uint4*>(plane + row * (BK * 2) + 16 * (c ^ swz(row))));
      };
#pragma unroll
      for (int sub = 0; sub < 2; sub++) {
        const int c = 4 * sl + 2 * sub + fc;
#pragma unroll
        for (int ni = 0; ni < kNi; ni++)
          fb[sub][ni] = frag(cur + plane_bytes, wn * kWc + ni * 32 + fr, c);
#pragma unroll
        for (int mi = 0; mi < 4; mi++) {
          if (mi >= live) break;
          fa[sub][mi] = frag(cur, rbase + mi * 32 + fr, c);
          if constexpr (SPLIT) fl[sub][mi] = frag(cur + 2 * plane_bytes, rbase + mi * 32 + fr, c);
        }
      }
      if (sl == kSps - 1) {
        // Stages issued: up to gi - 1; stage gc + 1 must have landed.
        if (gi - gc - 2 >= kDepth - 1)
          __builtin_amdgcn_s_waitcnt(vmcnt_only((kDepth - 1) * kLps));
        else
          __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      // ---- compute phase
#pragma unroll
      for (int sub = 0; sub < 2; sub++)
#pragma unroll
        for (int mi = 0; mi < 4; mi++) {
          if (mi >= live) break;
#pragma unroll
          for (int ni = 0; ni < kNi; ni++) {
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[sub][mi], fb[sub][ni],
                                                                  acc[mi][ni], 0, 0, 0);
            if constexpr (SPLIT)
              acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl[sub][mi], fb[sub][ni],
                                                                    acc[mi][ni], 0, 0, 0);
          }
        }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
    }
    gc++;
    if (++sc < ci.nk) continue;

    // ---- item kc done: store it, then move on.
    // Output element (mi, ni, r) of this lane: row rbase + 32 mi + 8 (r/4) +
    // 4 (lane/32) + r%4, column kWc wn + 32 ni + lane%32.
    const int wcol0 = ci.n0 + wn * kWc;
    if (wcol0 < ci.N) {
      if (GATEUP) {
        // Columns 64b .. 64b+63 of the wave are one (gate, up) block pair.
        uint16_t* h_hi = ci.routed ? P.h_hi : P.hs_hi;
        uint16_t* h_lo = ci.routed ? P.h_lo : P.hs_lo;
#pragma unroll
        for (int bp = 0; bp < kNi / 2; bp++) {
          if (wcol0 + 64 * bp >= ci.N) break;
          const int col = (wcol0 + 64 * bp) / 2 + fr;  // hidden column of this lane
#pragma unroll
          for (int mi = 0; mi < 4; mi++) {
            if (mi >= live) break;
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const int row = rbase + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
              if (row < ci.mrows) {
                const float gv = acc[mi][2 * bp][r];
                const float h = __fdividef(gv, 1.0f + __expf(-gv)) * acc[mi][2 * bp + 1][r];
                const size_t at = (size_t)(ci.base + ci.r0 + row) * ci.W + col;
                const uint16_t hb = bf16_bits(h);
                h_hi[at] = hb;
                if constexpr (SPLIT) h_lo[at] = bf16_bits(h - __uint_as_float((uint32_t)hb << 16));
              }
            }
          }
        }
      } else {
        float* out = ci.routed ? S.y : S.ys;
#pragma unroll
        for (int mi = 0; mi < 4; mi++) {
          if (mi >= live) break;
#pragma unroll
          for (int ni = 0; ni < kNi; ni++) {
            const int col = wcol0 + ni * 32 + fr;
            if (col >= ci.N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const int row = rbase + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
              if (row < ci.mrows) out[(size_t)(ci.base + ci.r0 + row) * L.H + col] = acc[mi][ni][r];
            }
          }
        }
      }
    }
    if (++kc == n_my) break;
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < kNi; ni++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.0f;
    sc = 0;
    ci = describe(kc);
    half = ci.mrows <= 128;
    rbase = half ? wm * 64 : wm * 128;
    live = __builtin_amdgcn_readfirstlane(min(half ? 2 : 4, max(0, (ci.mrows - rbase + 31) / 32)));
  }
  if (!grp) __syncthreads();
}

template <int BK, int NBUF, bool SPLIT>
constexpr size_t mfma_lds_bytes() {
  return (size_t)NBUF * (SPLIT ? 3 : 2) * kTileM * BK * sizeof(uint16_t) + 2 * kTileM * sizeof(int);
}
// BF16 activations: 64-deep stages (128-byte row segments, full cache
// lines per load), two buffers (128 KiB). FP32-class (hi + lo planes):
// 32-deep stages, three buffers (144 KiB). K is a multiple of 64 (hidden
// and expert widths).
constexpr int kBkBf16 = 64, kBufBf16 = 2;
constexpr int kBkSplit = 32, kBufSplit = 3;
constexpr int kWaves = 8;

template <bool SPLIT, bool GATEUP>
static const void* mfma_kernel() {
  if constexpr (SPLIT)
    return (const void*)mfma_group_kernel<kWaves, kBkSplit, kBufSplit, true, GATEUP>;
  else
    return (const void*)mfma_group_kernel<kWaves, kBkBf16, kBufBf16, false, GATEUP>;
}

template <bool SPLIT>
constexpr size_t mfma_lds() {
  return SPLIT ? mfma_lds_bytes<kBkSplit, kBufSplit, true>() : mfma_lds_bytes<kBkBf16, kBufBf16, false>();
}

void launch_split_planes(const float* x, size_t n, uint16_t* hi, uint16_t* lo, hipStream_t s) {
  if (n == 0) return;
  const size_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     s, x, n, hi, lo);
}

// Persistent grid: one workgroup per CU (the kernel holds a whole CU's LDS),
// a multiple of the XCD count; set by mfma_init_attributes.
static int g_mfma_grid = 256;

template <bool GATEUP>
static void launch_mfma(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, hipStream_t s) {
  (void)tiles_bound;
  const dim3 grid(g_mfma_grid);
  if (bf16_only)
    mfma_group_kernel<kWaves, kBkBf16, kBufBf16, false, GATEUP>
        <<<grid, dim3(kWaves * 64), mfma_lds<false>(), s>>>(L, S, P, T);
  else
    mfma_group_kernel<kWaves, kBkSplit, kBufSplit, true, GATEUP>
        <<<grid, dim3(kWaves * 64), mfma_lds<true>(), s>>>(L, S, P, T);
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
  const void* kernels[4] = {mfma_kernel<false, true>(), mfma_kernel<false, false>(),
                            mfma_kernel<true, true>(), mfma_kernel<true, false>()};
  const int lds[4] = {(int)mfma_lds<false>(), (int)mfma_lds<false>(), (int)mfma_lds<true>(),
                      (int)mfma_lds<true>()};
  for (int i = 0; i < 4; i++)
    (void)hipFuncSetAttribute(kernels[i], hipFuncAttributeMaxDynamicSharedMemorySize, lds[i]);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      cus >= kXcds)
    g_mfma_grid = cus / kXcds * kXcds;
  (void)hipGetLastError();  // a refused attribute surfaces at launch instead
}

}  // namespace uocr
