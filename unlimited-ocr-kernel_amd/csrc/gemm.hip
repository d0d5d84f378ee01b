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

// Split FP32 activations [rows, K] into bf16 hi and lo planes, k-blocked
// ([K/32][rows][32], as the GEMM reads them).
__global__ void split_planes_kernel(const float* __restrict__ x, int rows, int K,
                                    uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= (size_t)rows * K) return;
  const float4 v = *reinterpret_cast<const float4*>(x + i);
  const size_t t = i / K, k = i % K;
  const size_t o = ((k / 32) * rows + t) * 32 + k % 32;
  const float f[4] = {v.x, v.y, v.z, v.w};
  uint16_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    h[j] = bf16_bits(f[j]);
    l[j] = bf16_bits(f[j] - __uint_as_float((uint32_t)h[j] << 16));
  }
  *reinterpret_cast<uint2*>(hi + o) =
      make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
  if (lo)
    *reinterpret_cast<uint2*>(lo + o) =
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

// The same for 4 bytes per lane (lane l's dword lands at M0 + 4 l).
__device__ __forceinline__ void buffer_load_lds4(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
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

// A raw buffer resource over `bytes` bytes from `base` for stores: a store
// whose offset lies past the range is dropped by the hardware range check.
// Row offsets are passed through vgpr_offset, which keeps each whole in the
// VGPR offset (the compiler cannot split a constant part of it into the
// instruction or SGPR offset fields), so the check sees the full row.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t store_rsrc(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ int vgpr_offset(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt
// bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at maximum).
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// One work item: a TM x TN output tile of group g, rows r0.. of the group,
// columns n0... BF16 weights use two shapes: 256 x 256 (waves 2 x 4) for
// groups with more than 128 rows left, and 128 x 512 (waves 1 x 8) for the
// last tile of a group when at most 128 rows remain — a small group then
// streams its weights in fewer items without computing a mostly empty
// 256-row tile. A wave owns 128 rows x 64 columns (4 x 2 MFMA tiles).
//
// Q8: INT8-overlay weights, streamed as int8 rows with their block scales.
// Items are 64 x 512 (waves 1 x 8, each 64 x 64 as 2 x 2 MFMA tiles, the
// activations the first operand): an int8 weight is exact in bf16, so each
// 32-deep stage (one scale block) multiplies the activation planes by the
// int8 rows into a partial tile, and the block scale of each output row
// (lane-uniform in this layout) is applied to that partial with one FMA
// per element: the FP32 class needs the two activation terms only, BF16
// activations one. y is f32.
template <int TM, int BK, int NBUF, bool SPLIT, bool GATEUP, bool Q8>
__device__ __forceinline__ void mfma_item(const DeviceLayer& L, const Scratch& S,
                                          const MfmaPlanes& P, int T, int g, int r0, int n0,
                                          uint16_t* lds) {
  constexpr int WAVES = 8;
  static_assert(Q8 ? TM == 64 : (TM == 256 || TM == 128), "item shapes");
  constexpr int TN = Q8 ? 512 : 256 * 256 / TM;  // 256 or 512 (BF16); 512 (INT8)
  constexpr int kMi = TM >= 128 ? 4 : TM / 32;  // 32-row MFMA tiles per wave
  constexpr int kWr = 32 * kMi;            // rows per wave: 128, or 64 (INT8)
  constexpr int kWm = TM / kWr;            // wave rows
  constexpr int kWn = WAVES / kWm;         // wave columns
  constexpr int kWc = TN / kWn;            // 64 columns per wave
  constexpr int kNi = kWc / 32;
  const bool routed = g < L.E;
  const int W = L.width(g);
  const int N = GATEUP ? 2 * W : L.H;
  const int K = GATEUP ? L.H : W;
  const int group_rows = routed ? S.offsets[g + 1] - S.offsets[g] : T;
  const int mrows = min(TM, group_rows - r0);
  const int base = routed ? S.offsets[g] : 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / kWn, wn = wave % kWn;

  // Source row of tile row r (gate/up: the token, gathered through the
  // dispatch permutation; down: the dispatched row), -1 past the group.
  auto a_source = [&](int r) -> int {
    if (r >= mrows) return -1;
    if (GATEUP) return routed ? S.perm_rows[base + r0 + r] : r0 + r;
    return base + r0 + r;
  };

  // ---- LDS tiles. A stage holds the A plane(s) ([TM rows][BK] bf16) and
  // B: BF16 weights as a [TN rows][BK] bf16 plane; INT8 overlays (Q8) as
  // their int8 rows ([TN][BK] bytes, BK = 32: one scale block). Q8 block
  // scales arrive in groups of 8 blocks ([TN rows][8] f32, three group
  // buffers after the stage ring; see issue_scales). No padding: 16-byte chunk c of a bf16 row r
  // sits at position c ^ swz(r), which spreads the 16-byte fragment reads
  // of 16 consecutive rows over all LDS banks (int8 rows: c ^ ((r >> 3) & 1)
  // over their two chunks). Loads arrive as 1 KB wave segments (lane l ->
  // row l / chunks-per-row, position l % chunks-per-row).
  constexpr int kCpr = BK / 8;                 // 16-byte chunks per A row
  constexpr int kSegRows = 64 / kCpr;          // rows per 1 KB segment
  constexpr int kCprB = Q8 ? BK / 16 : kCpr;   // 16-byte chunks per B row
  constexpr int kSegRowsB = 64 / kCprB;
  static_assert(!Q8 || BK == 32, "INT8 stages are one 32-block deep");
  // Segments per wave and plane. When a plane has fewer segments than there
  // are waves (128 rows of 16-deep stages), waves past the last segment load
  // a copy of segment wave % count (the same bytes to the same place), so
  // every wave issues the same number of loads per stage.
  constexpr int kSegTotA = TM / kSegRows, kSegTotB = TN / kSegRowsB;
  constexpr int kSegA = kSegTotA >= WAVES ? kSegTotA / WAVES : 1;
  constexpr int kSegB = kSegTotB >= WAVES ? kSegTotB / WAVES : 1;
  static_assert(kSegTotA % WAVES == 0 || WAVES % kSegTotA == 0, "A segments");
  static_assert(kSegTotB % WAVES == 0 || WAVES % kSegTotB == 0, "B segments");
  const int segA0 = kSegTotA >= WAVES ? wave * kSegA : wave % kSegTotA;
  // Two A planes of WAVES / 2 segments each (64-row tiles, FP32 class):
  // waves 0..3 load the hi plane, waves 4..7 the lo plane, once each.
  constexpr bool kSplitA = SPLIT && 2 * kSegTotA == WAVES;
  const int segB0 = kSegTotB >= WAVES ? wave * kSegB : wave % kSegTotB;
  constexpr int kRowDiv = 16 / kCpr;
  auto swz = [](int r) { return (r / kRowDiv) % kCpr; };
  auto swzb = [&](int r) { return Q8 ? (r >> 3) & 1 : swz(r); };
  constexpr uint32_t a_plane = (uint32_t)TM * BK * 2;
  constexpr uint32_t b_plane = (uint32_t)TN * BK * (Q8 ? 1 : 2);
  constexpr int kAPlanes = SPLIT ? 2 : 1;
  constexpr uint32_t stage_bytes = kAPlanes * a_plane + b_plane;
  // Plane order in a stage: A hi, B, [A lo].
  constexpr uint32_t b_at = a_plane, alo_at = a_plane + b_plane;
  // Q8 scale groups: group q (blocks 8q .. 8q+7) in buffer q % 3.
  constexpr int kSGroup = 8;
  constexpr uint32_t sg_bytes = (uint32_t)TN * kSGroup * 4;
  constexpr uint32_t sg_at = (uint32_t)NBUF * stage_bytes;

  // Per-lane source offsets of this wave's segments (k = 0).
  const uint32_t row_bytes = (uint32_t)K * 2;
  const uint32_t row_bytes_b = (uint32_t)K * (Q8 ? 1 : 2);
  uint32_t a_off[kSegA], b_off[kSegB];
#pragma unroll
  for (int i = 0; i < kSegA; i++) {
    const int r = (segA0 + i) * kSegRows + lane / kCpr;
    const int c = (lane % kCpr) ^ swz(r);
    const int src_row = a_source(r);
    // The x planes and the h planes the gate/up epilogue writes are
    // k-blocked ([K/32][rows][32]: a stage's panel holds every row's 32 k).
    a_off[i] = src_row >= 0 ? (uint32_t)src_row * 64u + 16u * c : kDmaOut;
  }
#pragma unroll
  for (int i = 0; i < kSegB; i++) {
    const int r = (segB0 + i) * kSegRowsB + lane / kCprB;
    const int c = (lane % kCprB) ^ swzb(r);
    // Weights come from the k-blocked panels ([K/32][N][BK]): a stage's rows
    // are one contiguous run of N * BK elements.
    b_off[i] = n0 + r < N ? (uint32_t)(n0 + r) * (BK * (Q8 ? 1u : 2u)) + 16u * c : kDmaOut;
  }
  const int nblk = K / kQBlock;
  static_assert(!Q8 || TN == WAVES * 64, "a scale group is one dword load per wave and stage");
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
  // B: BF16 weights, or the INT8 overlay's int8 rows and block scales.
  const void* wmat;
  const float* wscale = nullptr;
  if constexpr (Q8) {
    wmat = GATEUP ? (const void*)(L.q13k + L.w13_offset(g)) : (const void*)(L.q2k + L.w2_offset(g));
    // Block scales block-major ([K/32][N] per group).
    wscale = GATEUP ? L.s13k + L.s13_offset(g) : L.s2k + L.s2_offset(g);
  } else {
    wmat = GATEUP ? (const void*)(L.w13k + L.w13_offset(g)) : (const void*)(L.w2k + L.w2_offset(g));
  }
  const i32x4 rs_a = buffer_rsrc(a_hi_src, a_rows * row_bytes);
  const i32x4 rs_l = buffer_rsrc(a_lo_src, a_rows * row_bytes);
  const i32x4 rs_b = buffer_rsrc(wmat, (uint32_t)N * row_bytes_b);
  const i32x4 rs_s = buffer_rsrc(Q8 ? (const void*)wscale : wmat, Q8 ? (uint32_t)N * nblk * 4u : 0u);
  const bool lo_wave = kSplitA && __builtin_amdgcn_readfirstlane(wave) >= WAVES / 2;
  const i32x4 rs_a1 = lo_wave ? rs_l : rs_a;
  // LDS byte addresses of this wave's first A and B segments of stage buffer 0.
  const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)lds);
  const uint32_t lds_a = __builtin_amdgcn_readfirstlane(lds_base + (uint32_t)segA0 * 1024u);
  const uint32_t lds_b = __builtin_amdgcn_readfirstlane(lds_base + b_at + (uint32_t)segB0 * 1024u);
  const uint32_t lds_a1 = lds_a + (lo_wave ? alo_at : 0u);
  // Q8 scales: part p (0..7) of group q is one dword load per wave, rows
  // 8 (8 p + wave) .. +7 with their 8 blocks (lane l: row + l / 8, blocks
  // 8 q ..). The source is block-major, so the 8 waves of one part read
  // 64 consecutive rows of each of the 8 blocks: whole 128-byte lines in
  // one stage (row-major rows had left each line to be read a quarter per
  // group, and refetched when it fell out of L2). Position j of row r holds block
  // 8 q + (j ^ sws(r)), so the 32 rows a half-wave reads for one block sit
  // in 32 distinct banks. Group q + 1 travels with the loads of stages
  // 8 q .. 8 q + 7 (part = stage % 8); group 0 before the first stage.
  // Group q + 1 overwrites group q - 2, whose last stage (8 q - 9) was read
  // before the loads of stage 8 q - kDepth are issued.
  auto sws = [](int r) { return (r >> 3) & 7; };
  auto issue_scales = [&](int q, int part) {
    const int r = (part * WAVES + wave) * 8 + lane / 8;
    const int blk = q * kSGroup + ((lane % 8) ^ sws(r));
    const uint32_t off = n0 + r < N && blk < nblk ? ((uint32_t)blk * N + n0 + r) * 4u : kDmaOut;
    const uint32_t dst = lds_base + sg_at + (uint32_t)(q % 3) * sg_bytes +
                         (uint32_t)(part * WAVES + wave) * 256u;
    buffer_load_lds4(rs_s, __builtin_amdgcn_readfirstlane(dst), off);
  };
  auto issue = [&](int buf, int k0) {
    const uint32_t st = (uint32_t)buf * stage_bytes;
    const uint32_t ka = (uint32_t)(k0 / 32) * a_rows * 64u;
    if constexpr (kSplitA) {
      buffer_load_lds16(rs_a1, lds_a1 + st, a_off[0] + ka);
    } else {
#pragma unroll
      for (int i = 0; i < kSegA; i++) {
        buffer_load_lds16(rs_a, lds_a + st + i * 1024u, a_off[i] + ka);
        if constexpr (SPLIT) buffer_load_lds16(rs_l, lds_a + st + alo_at + i * 1024u, a_off[i] + ka);
      }
    }
#pragma unroll
    for (int i = 0; i < kSegB; i++)
      buffer_load_lds16(rs_b, lds_b + st + i * 1024u, b_off[i] + (uint32_t)k0 * (Q8 ? 1u : 2u) * (uint32_t)N);
    if constexpr (Q8) {
      const int stage = k0 / BK;
      issue_scales(stage / kSGroup + 1, stage % kSGroup);
    }
  };

  floatx16 acc[kMi][kNi];
#pragma unroll
  for (int mi = 0; mi < kMi; mi++)
#pragma unroll
    for (int ni = 0; ni < kNi; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.0f;

  const int fr = lane & 31;   // fragment row / column
  const int fc = lane >> 5;   // fragment chunk inside a 16-wide k step
  const int nk = K / BK;

  // Q8: partial tiles of the current stage; the last one is folded with
  // last_scale during the next stage (zeros before the first).
  floatx16 part[Q8 ? kMi : 1][Q8 ? kNi : 1];
#pragma unroll
  for (int mi = 0; mi < (Q8 ? kMi : 1); mi++)
#pragma unroll
    for (int ni = 0; ni < (Q8 ? kNi : 1); ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) part[mi][ni][r] = 0.0f;
  float last_scale = 0.0f;

  // Q8 k order inside a 32-block: MFMA step s takes k = 16 fc + 8 s .. +7
  // from lane (fr, fc), so a lane's two steps are one 16-byte int8 chunk
  // (chunk fc of its row) and the activation fragments follow the same
  // order (bf16 chunk 2 fc + s). A block's partial is a sum over its 32 k
  // in any order.
  //
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
  constexpr int kDepth = NBUF - 1;
  constexpr int kLps = (kSplitA ? 1 : kSegA * kAPlanes) + kSegB + (Q8 ? 1 : 0);
  constexpr int kSub = BK / 16;
  const int grp = wave >> 2;
  // A wave whose columns all lie past N (the second half of a 512-wide
  // item over the last 256 columns: 2I = 1792 and H = 1280 are 3.5 and 2.5
  // such items) keeps its share of the loads and every barrier but reads
  // no fragments and issues no MFMAs; waves w and w + 4 share a SIMD, so
  // each SIMD keeps one busy wave.
  const bool wlive = (int)__builtin_amdgcn_readfirstlane(n0 + wn * kWc) < N;
  if constexpr (Q8)
    for (int part = 0; part < kSGroup; part++) issue_scales(0, part);
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
    bf16x8 fa[kSub][kMi], fl[kSub][SPLIT ? kMi : 1], fb[kSub][kNi];
    auto frag = [&](const char* plane, int row, int c) {
      return as_bf16x8(*reinterpret_cast<const uint4*>(plane + row * (BK * 2) + 16 * (c ^ swz(row))));
    };
    float bscale[kNi];
    uint4 qraw[kNi];
    if (wlive) {
      if constexpr (Q8) {
#pragma unroll
        for (int ni = 0; ni < kNi; ni++) {
          const int row = wn * kWc + ni * 32 + fr;
          bscale[ni] = *reinterpret_cast<const float*>(
              reinterpret_cast<const char*>(lds) + sg_at + (ks / kSGroup) % 3 * sg_bytes +
              row * (kSGroup * 4) + ((ks % kSGroup) ^ sws(row)) * 4);
          qraw[ni] = *reinterpret_cast<const uint4*>(cur + b_at + row * BK + 16 * (fc ^ swzb(row)));
        }
      }
#pragma unroll
      for (int sub = 0; sub < kSub; sub++) {
        const int c = Q8 ? 2 * fc + sub : 2 * sub + fc;
#pragma unroll
        for (int ni = 0; ni < kNi; ni++) {
          if constexpr (Q8) {
            // Eight int8 weights of row (output feature) wn*64 + 32 ni + fr,
            // k = 16 fc + 8 sub ..: |q| <= 127 is exact in bf16 (the f32 of a
            // small integer has zero low half), so the bf16 is its high half.
            const uint32_t lo = sub ? qraw[ni].z : qraw[ni].x;
            const uint32_t hi = sub ? qraw[ni].w : qraw[ni].y;
            uint32_t hp[4];
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
              const uint32_t word = j < 4 ? lo : hi;
              const int s0 = 8 * (j & 3), s1 = s0 + 8;
              const float w0 = (float)(int8_t)((word >> s0) & 0xffu);
              const float w1 = (float)(int8_t)((word >> s1) & 0xffu);
              hp[j / 2] = __builtin_amdgcn_perm(__float_as_uint(w1), __float_as_uint(w0), 0x07060302u);
            }
            fb[sub][ni] = as_bf16x8(make_uint4(hp[0], hp[1], hp[2], hp[3]));
          } else {
            fb[sub][ni] = frag(cur + b_at, wn * kWc + ni * 32 + fr, c);
          }
        }
#pragma unroll
        for (int mi = 0; mi < kMi; mi++) {
          fa[sub][mi] = frag(cur, wm * kWr + mi * 32 + fr, c);
          if constexpr (SPLIT) fl[sub][mi] = frag(cur + alo_at, wm * kWr + mi * 32 + fr, c);
        }
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
      c = GATEUP && !Q8 ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0)
                        : __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    };
    if (wlive) {
      if constexpr (Q8) {
        // Tile by tile: the stage's partial (one 32-block of K) of tile t,
        // while the block scales fold the partial of tile t - 1 into acc (one
        // FMA per element, the scale of this lane's output feature); tile 0
        // folds the previous stage's last tile, so only the last fold of the
        // item waits for its MFMAs.
        constexpr int kT = kMi * kNi;
#pragma unroll
        for (int t = 0; t < kT; t++) {
          const int mi = t / kNi, ni = t % kNi;
          floatx16 z = {};
          part[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[0][mi], fb[0][ni], z, 0, 0, 0);
          if constexpr (SPLIT) mma(fl[0][mi], fb[0][ni], part[mi][ni]);
#pragma unroll
          for (int sub = 1; sub < kSub; sub++) {
            mma(fa[sub][mi], fb[sub][ni], part[mi][ni]);
            if constexpr (SPLIT) mma(fl[sub][mi], fb[sub][ni], part[mi][ni]);
          }
          const int pt = (t + kT - 1) % kT, pmi = pt / kNi, pni = pt % kNi;
          const float sc = t == 0 ? last_scale : bscale[pni];
#pragma unroll
          for (int r = 0; r < 16; r++)
            acc[pmi][pni][r] = __builtin_fmaf(part[pmi][pni][r], sc, acc[pmi][pni][r]);
        }
        last_scale = bscale[kNi - 1];
        // One MFMA, then its share of the fold's FMAs (16 per tile), in turn.
#pragma unroll
        for (int i = 0; i < kT * kSub * kAPlanes; i++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 16 / (kSub * kAPlanes), 0);
        }
      } else {
#pragma unroll
        for (int sub = 0; sub < kSub; sub++)
#pragma unroll
          for (int mi = 0; mi < kMi; mi++)
#pragma unroll
            for (int ni = 0; ni < kNi; ni++) {
              mma(fa[sub][mi], fb[sub][ni], acc[mi][ni]);
              if constexpr (SPLIT) mma(fl[sub][mi], fb[sub][ni], acc[mi][ni]);
            }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  }
  if (!grp) __syncthreads();
  if constexpr (Q8) {
#pragma unroll
    for (int r = 0; r < 16; r++)
      acc[kMi - 1][kNi - 1][r] =
          __builtin_fmaf(part[kMi - 1][kNi - 1][r], last_scale, acc[kMi - 1][kNi - 1][r]);
  }

  const int wcol0 = n0 + wn * kWc;
  if constexpr (GATEUP && !Q8) {
    // Output element (mi, ni, r) of this lane: token row 128 wm + 32 mi +
    // lane%32, feature column kWc wn + 32 ni + 8 (r/4) + 4 (lane/32) + r%4;
    // registers 4j .. 4j+3 are four consecutive features of one token.
    // Columns 64b .. 64b+63 of the wave are one (gate, up) block pair: the
    // wave owns hidden block wn of the item, 32 columns.
    // SiLU(g) u = g / (1 + exp(-g)) u with a hardware reciprocal.
    //
    // h is staged in LDS (the stage ring is free after the loop) in the
    // layout of the k-blocked h planes ([W/32][rows][32]), then written out
    // per (plane, block) as one contiguous run of mrows x 64 bytes with full
    // 16-byte lanes, through a resource over exactly that run (rows >=
    // mrows are dropped). LDS: [plane][block][TM rows][64 B], the 16-byte
    // chunk c of row r at position c ^ ((r >> 2) & 3).
    static_assert(kNi == 2, "one (gate, up) block pair per wave");
    constexpr int kHB = TN / 64;                      // hidden blocks per item
    constexpr uint32_t kPlaneB = (uint32_t)kHB * TM * 64;  // 64 KiB
    static_assert(kAPlanes * kPlaneB <= (uint32_t)NBUF * stage_bytes, "h staging fits the ring");
    char* hst = reinterpret_cast<char*>(lds);
    auto hsw = [](int r) { return (r >> 2) & 3; };
    if (wcol0 < N) {
#pragma unroll
      for (int mi = 0; mi < kMi; mi++) {
        const int row = wm * kWr + 32 * mi + fr;
        char* rowp = hst + (uint32_t)wn * (TM * 64) + row * 64 + 8 * fc;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          float h[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float gv = acc[mi][0][4 * j + i];
            h[i] = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * acc[mi][1][4 * j + i];
          }
          // Two values per conversion (round to nearest even, as one at a
          // time): hi, then lo = bf16(h - hi) from hi's halves.
          const uint32_t hb01 = bf16_pair(h[0], h[1]), hb23 = bf16_pair(h[2], h[3]);
          const int pos = 16 * (j ^ hsw(row));
          *reinterpret_cast<uint2*>(rowp + pos) = make_uint2(hb01, hb23);
          if constexpr (SPLIT) {
            const uint32_t lb01 = bf16_pair(h[0] - __uint_as_float(hb01 << 16),
                                            h[1] - __uint_as_float(hb01 & 0xffff0000u));
            const uint32_t lb23 = bf16_pair(h[2] - __uint_as_float(hb23 << 16),
                                            h[3] - __uint_as_float(hb23 & 0xffff0000u));
            *reinterpret_cast<uint2*>(rowp + kPlaneB + pos) = make_uint2(lb01, lb23);
          }
        }
      }
    }
    __syncthreads();
    uint16_t* h_hi = routed ? P.h_hi : P.hs_hi;
    uint16_t* h_lo = routed ? P.h_lo : P.hs_lo;
    const size_t hrows = routed ? (size_t)T * L.K : (size_t)T;
    // 4 chunks per row, TM rows per (plane, block): a workgroup pass of 512
    // chunks covers half a square item's (plane, block) or a wide item's.
    constexpr int kChunks = kAPlanes * kHB * TM * 4;
    static_assert((TM * 4) % 512 == 0 || 512 % (TM * 4) == 0, "passes align with runs");
#pragma unroll
    for (int i = 0; i < kChunks / 512; i++) {
      const int pb = (512 * i) / (TM * 4);  // uniform: plane * kHB + block
      const int plane = pb / kHB, blk = pb % kHB;
      if (n0 + 64 * blk >= N) continue;
      const int within = tid + 512 * i - pb * TM * 4;
      const int row = within >> 2, c = within & 3;
      const uint4 v = *reinterpret_cast<const uint4*>(
          hst + (uint32_t)pb * (TM * 64) + row * 64 + 16 * (c ^ hsw(row)));
      uint16_t* run = (plane ? h_lo : h_hi) + ((size_t)(n0 / 64 + blk) * hrows + base + r0) * 32;
      const __amdgpu_buffer_rsrc_t rs = store_rsrc(run, (uint32_t)mrows * 64u);
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 d = {v.x, v.y, v.z, v.w};
      __builtin_amdgcn_raw_buffer_store_b128(d, rs, vgpr_offset(row * 64 + 16 * c), 0, 0);
    }
    return;
  }
  if (wcol0 >= N) return;
  if (GATEUP && Q8) {
    // Activations first: element (mi, ni, r) is token row 32 mi + 8 (r/4) +
    // 4 (lane/32) + r%4 and feature column wcol0 + 32 ni + lane%32; the
    // wave's 64 columns are one (gate, up) block pair, so ni = 0 holds the
    // gate values and ni = 1 the up values of hidden column wcol0/2 + lane%32.
    // The item's rows of that 32-column block of the k-blocked h planes
    // are one contiguous run of mrows x 64 bytes: stores go through a
    // resource over exactly that run (rows >= mrows are dropped).
    uint16_t* h_hi = routed ? P.h_hi : P.hs_hi;
    uint16_t* h_lo = routed ? P.h_lo : P.hs_lo;
    const size_t hrows = routed ? (size_t)T * L.K : (size_t)T;
    const size_t run = ((size_t)(wcol0 / 64) * hrows + base + r0) * 32;
    const __amdgpu_buffer_rsrc_t rs_hi = store_rsrc(h_hi + run, (uint32_t)mrows * 64u);
    const __amdgpu_buffer_rsrc_t rs_lo = store_rsrc(h_lo + run, (uint32_t)mrows * 64u);
    const int voff = (4 * fc) * 64 + 2 * fr;
#pragma unroll
    for (int mi = 0; mi < kMi; mi++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int off = vgpr_offset(voff + (mi * 32 + 8 * (r >> 2) + (r & 3)) * 64);
        const float gv = acc[mi][0][r];
        const float h = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * acc[mi][1][r];
        const uint16_t hb = bf16_bits(h);
        __builtin_amdgcn_raw_buffer_store_b16(hb, rs_hi, off, 0, 0);
        if constexpr (SPLIT)
          __builtin_amdgcn_raw_buffer_store_b16(bf16_bits(h - __uint_as_float((uint32_t)hb << 16)),
                                                rs_lo, off, 0, 0);
      }
  } else {
    // Output element (mi, ni, r) of this lane: row 128 wm + 32 mi + 8 (r/4)
    // + 4 (lane/32) + r%4, column kWc wn + 32 ni + lane%32.
    // FP32-class and INT8 weights: y in f32. BF16 weights with BF16
    // activations: y rounded to bf16 (the combine's operands), in the first
    // half of the same buffer.
    // Stores go through a resource over exactly the item's rows (rows >=
    // mrows fall past it and are dropped); a column >= N moves the lane's
    // offset past every resource.
    constexpr uint32_t esz = (SPLIT || Q8) ? 4 : 2;
    char* rows = reinterpret_cast<char*>(routed ? S.y : S.ys) + (size_t)(base + r0) * L.H * esz;
    const __amdgpu_buffer_rsrc_t rs = store_rsrc(rows, (uint32_t)mrows * L.H * esz);
    uint32_t voff[kNi];
#pragma unroll
    for (int ni = 0; ni < kNi; ni++) {
      const int col = wcol0 + ni * 32 + fr;
      voff[ni] = col < N ? ((uint32_t)(wm * kWr + 4 * fc) * L.H + col) * esz : kDmaOut;
    }
#pragma unroll
    for (int mi = 0; mi < kMi; mi++)
#pragma unroll
      for (int ni = 0; ni < kNi; ni++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int off = vgpr_offset(
              (int)(voff[ni] + (uint32_t)(mi * 32 + 8 * (r >> 2) + (r & 3)) * L.H * esz));
          if constexpr (SPLIT || Q8)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[mi][ni][r]), rs, off, 0, 0);
          else
            __builtin_amdgcn_raw_buffer_store_b16(bf16_bits(acc[mi][ni][r]), rs, off, 0, 0);
        }
  }
}


// Which variants run the 128 x 512 shape. The FP32-class BF16 engine moves
// as many bytes per stage in either shape (the A planes are hi + lo), so a
// small group's last tile costs half (12-layer 4096-token stack 7.21 -> 6.91
// ms; 1024 tokens 0.32 -> 0.27 ms). With one activation plane the wide
// stage moves 1.25x the bytes and a small group's items are bound by their
// weight stream from HBM, which the shape does not shorten: square items
// only are faster on the 4096-token stack (4.59 vs 4.69 ms), so BF16
// activations take the wide shape only up to kWideMaxTokens tokens, where
// small groups dominate. INT8 layers run 64-row tiles as 64 x 512 items
// only (512-token layer, FP32 class: 0.29 ms with 128 x 512 and 64 x 1024
// items of three product terms, 0.19 ms with these of two).
constexpr int kWideMaxTokens = 2048;

// Groups of one row are skipped when the overlay runs DynamicActivations
// (the batch engine's W8A8 path owns them). NBUF_W: stage buffers of the
// 128 x 512 shape.
// lists: bit 0 the shared expert's items, bit 1 the routed experts'. The
// shared expert's row tiles are [i * TM, ...) for TM the square items' rows
// (the dispatch's row tile), so a shared-only launch needs no dispatch.
template <int BK, int NBUF, int NBUF_W, bool SPLIT, bool GATEUP, bool Q8, bool WIDE>
__global__ __launch_bounds__(512, 1) void mfma_group_kernel(DeviceLayer L, Scratch S,
                                                            MfmaPlanes P, int T, int lists) {
  extern __shared__ __align__(16) uint16_t lds[];  // [stage ring][INT8 scale groups]
  static_assert(!Q8 || !WIDE, "INT8 items are 64 x 512 only");
  constexpr bool kWide = WIDE;

  // ---- work item. Workgroup ids reach the XCDs round-robin (id % 8), and
  // an XCD starts its workgroups in id order as its CUs free up. Five item
  // lists — the shared expert's items; the routed square items and the
  // small-group items (128 x 512) whose column tile is whole; then those
  // two kinds over a last, half-empty column tile (2I = 1792 and H = 1280
  // are 3.5 and 2.5 tiles of 512: half their waves idle, ~0.6 of an item) —
  // are each cut into 8 contiguous ranges of equal count, one per XCD. An
  // XCD runs its shared items first (in the down GEMM they are twice as
  // deep), then its whole-tile square items with its whole-tile small ones
  // spread evenly between them, then its half-tile items: the longest
  // first, so the round that ends the launch holds the shortest items.
  // Every XCD gets the same mix: a cost-weighted cut of one combined list
  // had put all the deeper shared items on the first two XCDs, whose
  // fewer, longer items then set the end of the launch (down span 177 us
  // against 147-159 us on the other XCDs). Neighbouring square items (same
  // expert, same rows) meet in one L2, and the weight streams of the small
  // groups (little reuse) spread over every XCD's path to HBM.
  // Tile lists (dispatch): routed [0, c2) square, [c2, c1) last tiles of
  // <= 128 rows (run as 128 x 512); a variant without the wide shape runs
  // them all as square items. The shared expert's tiles follow from T.
  constexpr int kSqTM = Q8 ? 64 : 256;
  const int shared_tiles = (lists & 1) ? (T + kSqTM - 1) / kSqTM : 0;
  const int routed_tiles = (lists & 2) ? S.counters[1] : 0;
  const int square_tiles = kWide && (lists & 2) ? S.counters[2] : routed_tiles;
  const int wide_tiles = routed_tiles - square_tiles;
  const int n_routed = GATEUP ? 2 * L.I : L.H;
  const int n_shared = GATEUP ? 2 * L.S : L.H;
  // INT8 layers: every tile is 64 rows, every item 64 x 512.
  constexpr int kItemN = Q8 ? 2 * kTileN : kTileN;
  const int nt_routed = (n_routed + kItemN - 1) / kItemN;
  const int nt_wide = (n_routed + 2 * kTileN - 1) / (2 * kTileN);
  const int nt_shared = (n_shared + kItemN - 1) / kItemN;
  // Column tiles past the last whole one (0 or 1 per row tile).
  const int half_sq = n_routed % kItemN != 0 && n_routed % kItemN <= kItemN / 2 ? 1 : 0;
  const int half_w = n_routed % (2 * kTileN) != 0 && n_routed % (2 * kTileN) <= kTileN ? 1 : 0;
  const int nf_sq = nt_routed - half_sq, nf_w = nt_wide - half_w;
  const long long shared_items = (long long)shared_tiles * nt_shared;
  const long long sqf_items = (long long)square_tiles * nf_sq;
  const long long wf_items = (long long)wide_tiles * nf_w;
  const long long sqh_items = (long long)square_tiles * half_sq;
  const long long wh_items = (long long)wide_tiles * half_w;
  auto cut = [](long long n, int x) { return n * x / kXcds; };  // XCD x's first of n
  const int xcd = blockIdx.x % kXcds;
  long long j = blockIdx.x / kXcds;
  const long long sh0 = cut(shared_items, xcd), n_sh = cut(shared_items, xcd + 1) - sh0;
  const long long sq0 = cut(sqf_items, xcd), n_sq = cut(sqf_items, xcd + 1) - sq0;
  const long long sm0 = cut(wf_items, xcd), n_sm = cut(wf_items, xcd + 1) - sm0;
  const long long hq0 = cut(sqh_items, xcd), n_hq = cut(sqh_items, xcd + 1) - hq0;
  const long long hw0 = cut(wh_items, xcd), n_hw = cut(wh_items, xcd + 1) - hw0;
  if (j >= n_sh + n_sq + n_sm + n_hq + n_hw) return;
  int tile = -1, ntile, g, r0;
  bool take_small = false;
  // Slot r of n_a + n_b slots interleaving two lists: the b item index when
  // floor(r n_b / n) steps (b items spread evenly), else the a index.
  auto spread = [](long long r, long long n_a, long long n_b, bool& is_b) {
    const long long b_before = r * n_b / (n_a + n_b);
    is_b = (r + 1) * n_b / (n_a + n_b) > b_before;
    return is_b ? b_before : r - b_before;
  };
  if (j < n_sh) {
    const long long item = sh0 + j;
    g = L.E;
    r0 = (int)(item / nt_shared) * kSqTM;
    ntile = (int)(item % nt_shared);
  } else if ((j -= n_sh) < n_sq + n_sm) {
    // The small-group items spread between the square ones, so the
    // HBM-bound weight streams of small groups run alongside the
    // L2-resident square work instead of all at once.
    const long long i = spread(j, n_sq, n_sm, take_small);
    if (take_small) {
      tile = square_tiles + (int)((sm0 + i) / nf_w);
      ntile = (int)((sm0 + i) % nf_w);
    } else {
      tile = (int)((sq0 + i) / nf_sq);
      ntile = (int)((sq0 + i) % nf_sq);
    }
  } else {
    const long long i = spread(j - n_sq - n_sm, n_hq, n_hw, take_small);
    if (take_small) {
      tile = square_tiles + (int)(hw0 + i);
      ntile = nt_wide - 1;
    } else {
      tile = (int)(hq0 + i);
      ntile = nt_routed - 1;
    }
  }
  if (tile >= 0) {
    g = S.tiles[2 * tile];
    r0 = S.tiles[2 * tile + 1];
  }
  if (Q8 && g < L.E && L.quant_mode == kQuantDynamic &&
      S.offsets[g + 1] - S.offsets[g] == 1)
    return;
  if constexpr (kWide) {
    if (take_small) {
      mfma_item<128, BK, NBUF_W, SPLIT, GATEUP, false>(L, S, P, T, g, r0, ntile * 2 * kTileN,
                                                       lds);
      return;
    }
  }
  mfma_item<Q8 ? 64 : 256, BK, NBUF, SPLIT, GATEUP, Q8>(L, S, P, T, g, r0, ntile * kItemN, lds);
}

// Dynamic LDS of one shape: NBUF stages of the A planes (TM rows, bf16) and
// B (256 * 256 / TM rows of bf16, or 512 of int8), BK deep; INT8 also holds
// three scale groups (512 rows x 8 blocks, f32).
constexpr size_t stage_lds(int TM, int BK, int NBUF, int a_planes, bool q8) {
  const size_t tn = q8 ? 2 * (size_t)kTileN : (size_t)kTileM * kTileN / TM;
  return (size_t)NBUF * ((size_t)a_planes * TM * BK * 2 + tn * BK * (q8 ? 1 : 2)) +
         (q8 ? 3 * tn * 8 * 4 : 0);  // Q8: three scale groups of 8 blocks
}
template <int BK, int NBUF, int NBUF_W, int AP, bool Q8, bool WIDE>
constexpr size_t mfma_lds_bytes() {
  const size_t sq = stage_lds(Q8 ? 64 : 256, BK, NBUF, AP, Q8);
  const size_t wd = WIDE ? stage_lds(128, BK, NBUF_W, AP, Q8) : 0;
  return sq > wd ? sq : wd;
}
// BF16 activations: 32-deep stages, four buffers (128 KiB), three for the
// 128 x 512 items of its small-batch variant (120 KiB). FP32-class (hi +
// lo planes): 32-deep stages, three buffers (144 KiB either shape). INT8
// overlay, 64 x 512 items (20 / 24 KiB per stage): 32-deep stages (one
// scale block), four buffers, plus 48 KiB of scale groups (128 / 144 KiB).
constexpr int kBkBf16 = 32, kBufBf16 = 4, kBufBf16W = 3, kBkSplit = 32, kBufSplit = 3;
constexpr int kBkQ = 32, kBufQ = 4;

void launch_split_planes(const float* x, int rows, int K, uint16_t* hi, uint16_t* lo,
                         hipStream_t s) {
  if (rows <= 0) return;
  const size_t threads = ((size_t)rows * K + 3) / 4;
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     s, x, rows, K, hi, lo);
}

// Workgroups: 8 XCDs times the most items one XCD can take. Items are
// bounded by every row tile times the widest column count of its items (a
// 128 x 512 item replaces two square ones; INT8 layers: 512 columns); an
// XCD takes an eighth of each of five lists, so at most bound / 8 + 5.
static unsigned mfma_grid(const DeviceLayer& L, int tiles_bound, bool gateup) {
  const int n = gateup ? std::max(2 * L.S, 2 * L.I) : L.H;
  const int item_n = L.quant_mode != kQuantNone ? 2 * kTileN : kTileN;  // INT8: 64 x 512
  const long long items = (long long)tiles_bound * ((n + item_n - 1) / item_n);
  // An XCD takes an eighth of each of its five lists, each rounded up.
  const long long per_xcd = (items + kXcds - 1) / kXcds + 5;
  return (unsigned)(per_xcd * kXcds);
}

#define UOCR_MFMA_KERNEL(BK, NBUF, NBUFW, SPLIT, GATEUP, Q8, WIDE) \
  mfma_group_kernel<BK, NBUF, NBUFW, SPLIT, GATEUP, Q8, WIDE>
#define UOCR_MFMA_LDS(BK, NBUF, NBUFW, AP, Q8, WIDE) mfma_lds_bytes<BK, NBUF, NBUFW, AP, Q8, WIDE>()

template <bool GATEUP>
static void launch_mfma(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, int lists, hipStream_t s) {
  const dim3 grid(mfma_grid(L, tiles_bound, GATEUP)), block(512);
  if (L.quant_mode != kQuantNone) {
    if (bf16_only)
      UOCR_MFMA_KERNEL(kBkQ, kBufQ, kBufQ, false, GATEUP, true, false)
          <<<grid, block, UOCR_MFMA_LDS(kBkQ, kBufQ, kBufQ, 1, true, false), s>>>(L, S, P, T, lists);
    else
      UOCR_MFMA_KERNEL(kBkQ, kBufQ, kBufQ, true, GATEUP, true, false)
          <<<grid, block, UOCR_MFMA_LDS(kBkQ, kBufQ, kBufQ, 2, true, false), s>>>(L, S, P, T, lists);
  } else if (bf16_only && T <= kWideMaxTokens) {
    UOCR_MFMA_KERNEL(kBkBf16, kBufBf16, kBufBf16W, false, GATEUP, false, true)
        <<<grid, block, UOCR_MFMA_LDS(kBkBf16, kBufBf16, kBufBf16W, 1, false, true), s>>>(L, S,
                                                                                         P, T, lists);
  } else if (bf16_only) {
    UOCR_MFMA_KERNEL(kBkBf16, kBufBf16, kBufBf16W, false, GATEUP, false, false)
        <<<grid, block, UOCR_MFMA_LDS(kBkBf16, kBufBf16, kBufBf16W, 1, false, false), s>>>(L, S,
                                                                                          P, T, lists);
  } else {
    UOCR_MFMA_KERNEL(kBkSplit, kBufSplit, kBufSplit, true, GATEUP, false, true)
        <<<grid, block, UOCR_MFMA_LDS(kBkSplit, kBufSplit, kBufSplit, 2, false, true), s>>>(L, S,
                                                                                           P, T, lists);
  }
}

void launch_mfma_gateup(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                        int tiles_bound, bool bf16_only, int lists, hipStream_t s) {
  launch_mfma<true>(L, S, P, T, tiles_bound, bf16_only, lists, s);
}

void launch_mfma_down(const DeviceLayer& L, const Scratch& S, const MfmaPlanes& P, int T,
                      int tiles_bound, bool bf16_only, int lists, hipStream_t s) {
  launch_mfma<false>(L, S, P, T, tiles_bound, bf16_only, lists, s);
}

// One 16-byte chunk per thread: chunk c of (matrix, block kb, row n).
__global__ __launch_bounds__(256) void panelize_kernel(const uint4* __restrict__ in, uint4* __restrict__ out,
                                                       int N, int K, int cpb, size_t total) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const size_t per_matrix = (size_t)N * (K / 32) * cpb;  // chunks per matrix
  const size_t m = i / per_matrix, rest = i % per_matrix;
  const size_t kb = rest / ((size_t)N * cpb), n = (rest / cpb) % N, c = rest % cpb;
  // Source: row n, elements 32 kb .. (chunk c); K / 32 * cpb chunks per row.
  out[i] = in[m * per_matrix + n * (size_t)(K / 32) * cpb + kb * cpb + c];
}

__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ in,
                                                            float* __restrict__ out, int rows,
                                                            int cols, size_t total) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const size_t per = (size_t)rows * cols;
  const size_t m = i / per, rest = i % per;
  const size_t r = rest / cols, c = rest % cols;
  out[m * per + c * rows + r] = in[i];
}

void launch_transpose_f32(const float* in, float* out, int rows, int cols, int groups,
                          hipStream_t s) {
  if (rows <= 0 || cols <= 0 || groups <= 0) return;
  const size_t total = (size_t)groups * rows * cols;
  hipLaunchKernelGGL(transpose_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     in, out, rows, cols, total);
}

void launch_panelize(const void* in, void* out, int elem_bytes, int N, int K, int groups,
                     hipStream_t s) {
  if (N <= 0 || K <= 0 || groups <= 0) return;
  const int cpb = 32 * elem_bytes / 16;  // 16-byte chunks per 32-element block
  const size_t total = (size_t)groups * N * (K / 32) * cpb;
  hipLaunchKernelGGL(panelize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     (const uint4*)in, (uint4*)out, N, K, cpb, total);
}

void mfma_init_attributes() {
  auto set = [](const void* k, size_t bytes) {
    (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  };
#define UOCR_MFMA_ATTR(BK, NBUF, NBUFW, SPLIT, Q8, AP, WIDE)                                \
  set((const void*)UOCR_MFMA_KERNEL(BK, NBUF, NBUFW, SPLIT, true, Q8, WIDE),              \
      UOCR_MFMA_LDS(BK, NBUF, NBUFW, AP, Q8, WIDE));                                      \
  set((const void*)UOCR_MFMA_KERNEL(BK, NBUF, NBUFW, SPLIT, false, Q8, WIDE),             \
      UOCR_MFMA_LDS(BK, NBUF, NBUFW, AP, Q8, WIDE));
  UOCR_MFMA_ATTR(kBkBf16, kBufBf16, kBufBf16W, false, false, 1, false)
  UOCR_MFMA_ATTR(kBkBf16, kBufBf16, kBufBf16W, false, false, 1, true)
  UOCR_MFMA_ATTR(kBkSplit, kBufSplit, kBufSplit, true, false, 2, true)
  UOCR_MFMA_ATTR(kBkQ, kBufQ, kBufQ, false, true, 1, false)
  UOCR_MFMA_ATTR(kBkQ, kBufQ, kBufQ, true, true, 2, false)
#undef UOCR_MFMA_ATTR
  (void)hipGetLastError();  // a refused attribute surfaces at launch instead
}

}  // namespace uocr
