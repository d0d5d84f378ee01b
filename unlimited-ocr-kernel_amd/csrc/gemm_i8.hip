// Int8 x int8 grouped GEMM with int32 block accumulation: the opt-in
// UOCR_FLAG_INT8_MFMA mode of DynamicActivations layers. An extension: the
// reference quantises the activations of single-row groups only
// (src/decoder/mod.rs:103-104); this mode gives every group, of any row
// count, the arithmetic of Int8Matrix::linear_dynamic_int8
// (src/cpu/quantized.rs:155-236) row by row:
//   x -> per 32-block int8 with scale xs (Int8Matrix::quantize, :43-74);
//   y[n] = sum_b ((sum_{i in b} w[n,i] * x[i] as i32) as f32 * ws[n,b]) * xs[b].
// The int32 block sums come from v_mfma_i32_32x32x32_i8, one instruction per
// 32 x 32 output tile and 32-deep K block (a scale block), so they are exact
// and equal the reference's bit for bit; the scaled products are added over
// the blocks in ascending order as the reference does, each multiply and add
// separately rounded.
//
// A workgroup of 4 waves computes a 64-row item of one expert group: the
// weight rows are the MFMA's first operand, so a lane holds one token and 16
// output features per 32 x 32 tile. Gate/up items are 256 columns wide and
// wave w's 64 columns are one (gate, up) block pair of the interleaved w13
// rows (SiLU(g) * u is register-local); down items are 128 columns wide, 32
// per wave. Each 32-deep stage (int8 rows of the token tile and of the
// weight tile, and their f32 block scales) is brought into LDS by
// global->LDS loads, NST stages ahead.
#include "common.hpp"
#include "moe_kernels.hpp"
#include "rowdot.hpp"

namespace uocr {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kI8TileM = 64;   // token rows per item
// Output features per item: 256 for gate/up (each wave one gate/up block
// pair), 128 for down (each wave one 32-feature tile), so the down launch's
// items are short enough that the shared expert's (twice as deep) do not
// set its end.
constexpr int i8_nft(bool gateup) { return gateup ? 2 : 1; }  // feature tiles per wave
constexpr int i8_tile_n(bool gateup) { return 128 * i8_nft(gateup); }
constexpr int kI8Stages = 4;   // LDS ring depth
constexpr int kI8Threads = 256;
constexpr int kI8Xcds = 8;

// Stage layout (bytes): token rows [64][32], weight rows [256][32], token
// scales [64] f32, weight scales [256] f32. Row chunk c (16 B) of row r sits
// at position c ^ ((r >> 3) & 1), so the 16-byte fragment reads of 16
// consecutive rows cover all LDS banks.
constexpr uint32_t kI8ARows = kI8TileM * 32;
constexpr uint32_t i8_brows(bool gateup) { return (uint32_t)i8_tile_n(gateup) * 32; }
constexpr uint32_t kI8AScale = kI8TileM * 4;
constexpr uint32_t i8_stage(bool gateup) {  // 11.5 KB (gate/up), 6.75 KB (down)
  return kI8ARows + i8_brows(gateup) + kI8AScale + (uint32_t)i8_tile_n(gateup) * 4;
}

__device__ __forceinline__ i32x4 i8_rsrc(const void* base, uint32_t bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  i32x4 r;
  r.x = (int)(uint32_t)a;
  r.y = (int)((a >> 32) & 0xffffu);
  r.z = (int)bytes;
  r.w = 0x00020000;
  return r;
}

// Global -> LDS (lane l's bytes land at M0 + size * l); range-checked.
__device__ __forceinline__ void i8_load16(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory");
}
__device__ __forceinline__ void i8_load4(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory");
}

constexpr uint32_t kI8Out = 0x80000000u;  // offset past every resource

constexpr int i8_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Loads issued per wave per stage: token rows 2 KB = 2 wave loads, weight
// rows 8 KB = 8, token scales 1, weight scales 4: 15 over 4 waves, waves
// 0..2 take 4 and wave 3 takes 3 (+1 repeated token-scale load so every
// wave issues 4).
// Wave-loads per stage: token rows 2, weight rows 4 per feature tile pair
// member, token scales 1, weight scales 2 per 128 features; gate/up 15
// (4 per wave, the 16th repeats the token-scale load), down 9 (3 per wave,
// three repeats).
constexpr int i8_loads(bool gateup) { return 3 + 6 * i8_nft(gateup); }
constexpr int i8_loads_per_wave(bool gateup) { return (i8_loads(gateup) + 3) / 4; }
constexpr int i8_wg_per_cu(bool gateup) { return gateup ? 3 : 4; }

// Row of w13 (interleaved in blocks of 32: gate j.., up j..) -> its row in
// checkpoint order (gate rows 0..W-1, then up rows W..2W-1).
__device__ __forceinline__ int ckpt_row13(int r, int W) {
  const int blk = r >> 6, in = r & 63;
  return in < 32 ? 32 * blk + in : W + 32 * blk + (in - 32);
}

}  // namespace

// Items: (row tile, column tile), routed tiles first, column tile fastest;
// workgroup ids reach the XCDs round-robin and are remapped so each XCD
// takes a contiguous range (an expert's items share one L2).
// TRACE: the instantiation that also stores every block sum (tests); the
// plain one carries no trace code, so it fits three workgroups per CU.
template <bool GATEUP, bool TRACE>
__global__ __launch_bounds__(kI8Threads, i8_wg_per_cu(GATEUP)) void i8_group_kernel(DeviceLayer L,
                                                                          Scratch S, I8Planes P,
                                                                          int T) {
  extern __shared__ __align__(16) char lds[];
  constexpr int NFT = i8_nft(GATEUP), kTileN = i8_tile_n(GATEUP);
  constexpr int kLoads = i8_loads(GATEUP), kLpw = i8_loads_per_wave(GATEUP);
  constexpr uint32_t kStage = i8_stage(GATEUP), kBAt = kI8ARows,
                     kASAt = kI8ARows + i8_brows(GATEUP), kBSAt = kASAt + kI8AScale;
  const int all_tiles = S.counters[0];
  const int routed_tiles = S.counters[1];
  const int n_routed = GATEUP ? 2 * L.I : L.H;
  const int n_shared = GATEUP ? 2 * L.S : L.H;
  const int nt_r = (n_routed + kTileN - 1) / kTileN;
  const int nt_s = (n_shared + kTileN - 1) / kTileN;
  const int items = routed_tiles * nt_r + (all_tiles - routed_tiles) * nt_s;
  const int per_xcd = (items + kI8Xcds - 1) / kI8Xcds;
  const int item = (blockIdx.x % kI8Xcds) * per_xcd + blockIdx.x / kI8Xcds;
  if ((int)(blockIdx.x / kI8Xcds) >= per_xcd || item >= items) return;
  int tile, ntile;
  if (item < routed_tiles * nt_r) {
    tile = item / nt_r;
    ntile = item % nt_r;
  } else {
    const int i = item - routed_tiles * nt_r;
    tile = routed_tiles + i / nt_s;
    ntile = i % nt_s;
  }
  const int g = S.tiles[2 * tile], r0 = S.tiles[2 * tile + 1];
  const bool routed = g < L.E;
  const int W = L.width(g);
  const int N = GATEUP ? 2 * W : L.H;
  const int K = GATEUP ? L.H : W;
  const int nblk = K / kQBlock;
  const int group_rows = routed ? S.offsets[g + 1] - S.offsets[g] : T;
  const int mrows = min(kI8TileM, group_rows - r0);
  const int base = routed ? S.offsets[g] : 0;
  const int n0 = ntile * kTileN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar load plan

  // ---- sources. Token rows: gate/up reads the quantised layer input
  // (routed rows gathered through the dispatch permutation), down reads the
  // quantised hidden rows (dispatched order; shared rows after the routed).
  const int8_t* aq;
  const float* as;
  uint32_t a_rows, a_row0;
  if (GATEUP) {
    aq = P.xq;
    as = P.xs;
    a_rows = (uint32_t)T;
    a_row0 = 0;
  } else {
    aq = routed ? P.hid_q : P.hid_q + (size_t)T * L.K * L.I;
    as = routed ? P.hid_s : P.hid_s + (size_t)T * L.K * (L.I / kQBlock);
    a_rows = routed ? (uint32_t)T * L.K : (uint32_t)T;
    a_row0 = (uint32_t)(base + r0);
  }
  // Weights from the k-blocked panels ([K/32][N][32] per group): stage b's
  // 32 bytes of the tile's rows are one contiguous run, so every 128-byte
  // line is read whole in one stage (row-major rows left each line to be
  // read a quarter per stage, and refetched when it fell out of L2).
  const int8_t* bq = GATEUP ? L.q13k + L.w13_offset(g) : L.q2k + L.w2_offset(g);
  // Block scales block-major ([K/32][N] per group): one stage's scales of
  // the tile's rows are one contiguous run.
  const float* bs = GATEUP ? L.s13k + L.s13_offset(g) : L.s2k + L.s2_offset(g);
  const uint32_t bs_row = 4u, bs_blk = (uint32_t)N * 4u;  // bytes per row, per block
  const i32x4 rs_aq = i8_rsrc(aq, a_rows * (uint32_t)K);
  const i32x4 rs_as = i8_rsrc(as, a_rows * (uint32_t)nblk * 4u);
  const i32x4 rs_bq = i8_rsrc(bq, (uint32_t)N * (uint32_t)K);
  const i32x4 rs_bs = i8_rsrc(bs, (uint32_t)N * (uint32_t)nblk * 4u);
  auto a_source = [&](int r) -> int {
    if (r >= mrows) return -1;
    if (GATEUP) return routed ? S.perm_rows[base + r0 + r] : r0 + r;
    return (int)a_row0 + r;
  };

  // Per-lane load plan of this wave (4 wave-loads per stage): global byte
  // offsets at block 0 and the LDS position of each.
  uint32_t off[kLpw], lds_at[kLpw];
  int kind[kLpw];  // 0 token rows, 1 weight rows, 2 token scales, 3 weight scales
#pragma unroll
  for (int j = 0; j < kLpw; j++) {
    constexpr int kNB = 4 * NFT;  // weight-row wave-loads
    const int slot = wave * kLpw + j;  // slots past kLoads repeat the token-scale load
    const int ld = slot < kLoads ? slot : 2 + kNB;
    if (ld < 2) {  // token rows: 32 rows of 32 B per wave-load
      const int r = ld * 32 + lane / 2, c = (lane & 1) ^ ((r >> 3) & 1);
      const int src = a_source(r);
      kind[j] = 0;
      off[j] = src >= 0 ? (uint32_t)src * (uint32_t)K + 16u * c : kI8Out;
      lds_at[j] = (uint32_t)ld * 1024u;
    } else if (ld < 2 + kNB) {  // weight rows
      const int r = (ld - 2) * 32 + lane / 2, c = (lane & 1) ^ ((r >> 3) & 1);
      kind[j] = 1;
      off[j] = n0 + r < N ? (uint32_t)(n0 + r) * 32u + 16u * c : kI8Out;
      lds_at[j] = kBAt + (uint32_t)(ld - 2) * 1024u;
    } else if (ld == 2 + kNB) {  // token scales: 64 rows, one dword each
      const int src = a_source(lane);
      kind[j] = 2;
      off[j] = src >= 0 ? (uint32_t)src * (uint32_t)nblk * 4u : kI8Out;
      lds_at[j] = kASAt;
    } else {  // weight scales: 4 x 64 rows
      const int r = (ld - 3 - kNB) * 64 + lane;
      kind[j] = 3;
      off[j] = n0 + r < N ? (uint32_t)(n0 + r) * bs_row : kI8Out;
      lds_at[j] = kBSAt + (uint32_t)(ld - 3 - kNB) * 256u;
    }
  }
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)lds);
  auto issue = [&](int stage, int b) {
    const uint32_t st = lds0 + (uint32_t)stage * kStage;
#pragma unroll
    for (int j = 0; j < kLpw; j++) {
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(st + lds_at[j]);
      const bool out = off[j] == kI8Out;
      if (kind[j] == 0) i8_load16(rs_aq, m0, out ? kI8Out : off[j] + 32u * b);
      else if (kind[j] == 1) i8_load16(rs_bq, m0, out ? kI8Out : off[j] + 32u * N * b);
      else if (kind[j] == 2) i8_load4(rs_as, m0, out ? kI8Out : off[j] + 4u * b);
      else i8_load4(rs_bs, m0, out ? kI8Out : off[j] + bs_blk * b);
    }
  };

  // Accumulators: [feature tile ft][token tile tt]; lane l holds token
  // 32 tt + l % 32 and features 32 ft + 8 (r / 4) + 4 (l / 32) + r % 4 of the
  // wave's 64 columns.
  float acc[NFT][2][16];
#pragma unroll
  for (int ft = 0; ft < NFT; ft++)
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[ft][tt][r] = -0.0f;  // Rust's float sum starts at -0.0

  const int fr = lane & 31, fc = lane >> 5;
  const int wcol = wave * 32 * NFT;  // this wave's first feature within the item
  // Trace of the exact block sums (tests): routed rows by dispatched
  // position, the shared expert's only when it has a single row.
  int32_t* trace = nullptr;
  if constexpr (TRACE) {
    if (routed) trace = GATEUP ? S.q8.gateup : S.q8.down;
    else if (T == 1) trace = GATEUP ? S.q8.s_gateup : S.q8.s_down;
  }

  constexpr int kDepth = kI8Stages - 1;
  for (int i = 0; i < kDepth; i++)
    if (i < nblk) issue(i, i);
  for (int b = 0; b < nblk; b++) {
    // Stage b landed (own loads: the later stages still in flight), then the
    // barrier publishes every wave's part and retires stage b - 1's readers.
    const int ahead = min(kDepth - 1, nblk - 1 - b);
    if (ahead >= 2) __builtin_amdgcn_s_waitcnt(i8_vmcnt(2 * kLpw));
    else if (ahead == 1) __builtin_amdgcn_s_waitcnt(i8_vmcnt(kLpw));
    else __builtin_amdgcn_s_waitcnt(i8_vmcnt(0));
    __syncthreads();
    if (b + kDepth < nblk) issue((b + kDepth) % kI8Stages, b + kDepth);
    const char* cur = lds + (b % kI8Stages) * kStage;
    i32x4 wf[NFT], xf[2];
#pragma unroll
    for (int ft = 0; ft < NFT; ft++) {
      const int r = wcol + 32 * ft + fr;
      wf[ft] = *reinterpret_cast<const i32x4*>(cur + kBAt + r * 32 + 16 * (fc ^ ((r >> 3) & 1)));
    }
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
      const int r = 32 * tt + fr;
      xf[tt] = *reinterpret_cast<const i32x4*>(cur + r * 32 + 16 * (fc ^ ((r >> 3) & 1)));
    }
    float xsv[2];
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
      xsv[tt] = *reinterpret_cast<const float*>(cur + kASAt + (32 * tt + fr) * 4);
#pragma unroll
    for (int ft = 0; ft < NFT; ft++) {
      // This feature tile's 16 weight scales (lane features 8 q + 4 fc + 0..3).
      float wsv[16];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 v = *reinterpret_cast<const float4*>(
            cur + kBSAt + (wcol + 32 * ft + 8 * q + 4 * fc) * 4);
        wsv[4 * q + 0] = v.x;
        wsv[4 * q + 1] = v.y;
        wsv[4 * q + 2] = v.z;
        wsv[4 * q + 3] = v.w;
      }
      // Both token tiles' products issued before either fold, so one
      // MFMA runs while the other's sums are scaled (the compiler otherwise
      // serialises them on one result register set).
      i32x16 p[2];
#pragma unroll
      for (int tt = 0; tt < 2; tt++)
        p[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[ft], xf[tt], i32x16{}, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        const i32x16 pv = p[tt];
#pragma unroll
        for (int r = 0; r < 16; r++)
          acc[ft][tt][r] = acc[ft][tt][r] + ((float)pv[r] * wsv[r]) * xsv[tt];
        if (TRACE && trace) {
          const int row = 32 * tt + fr;
          if (row < mrows) {
            const size_t pos = routed ? (size_t)(base + r0 + row) : 0;
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const int n = n0 + wcol + 32 * ft + 8 * (r >> 2) + 4 * fc + (r & 3);
              if (n >= N) continue;
              const int cr = GATEUP ? ckpt_row13(n, W) : n;
              trace[(pos * (size_t)N + cr) * nblk + b] = pv[r];
            }
          }
        }
      }
    }
  }

  // ---- epilogue
  const int row_in = fr;  // token within a token tile
  if constexpr (GATEUP) {
    // Feature tile 0 holds gate values, tile 1 the matching up values:
    // hidden column 32 (n0 + wcol) / 64 + 8 (r/4) + 4 fc + r%4.
    if (n0 + wcol >= N) return;
    const int hcol0 = (n0 + wcol) / 2;
    if constexpr (TRACE) {
      // FP32 hidden rows (the trace copies them), quantised by their own
      // launch.
      float* hout = routed ? P.hid : P.hid_shared;
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        const int row = 32 * tt + row_in;
        if (row >= mrows) continue;
        const size_t at = routed ? (size_t)(base + r0 + row) * L.I : (size_t)(r0 + row) * L.S;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int col = hcol0 + 8 * (r >> 2) + 4 * fc + (r & 3);
          hout[at + col] = silu(acc[0][tt][r]) * acc[1][tt][r];
        }
      }
    } else {
      // Int8Matrix::quantize (src/cpu/quantized.rs:43-74) of the hidden
      // rows here, as quantize_rows_kernel does it: a wave's 32 hidden
      // values of a token row are one 32-block (hcol0 is a multiple of 32),
      // 16 in lane l and 16 in lane l ^ 32.
      const int W = L.width(g);
      const int nb = W / kQBlock, blk = hcol0 / kQBlock;
      int8_t* qbase = routed ? P.hid_q : P.hid_q + (size_t)T * L.K * L.I;
      float* sbase = routed ? P.hid_s : P.hid_s + (size_t)T * L.K * (L.I / kQBlock);
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        const int row = 32 * tt + row_in;
        float h[16];
        float maximum = 0.0f;
        int bad = 0;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          h[r] = silu(acc[0][tt][r]) * acc[1][tt][r];
          bad |= !isfinite(h[r]);
          maximum = fmaxf(maximum, fabsf(h[r]));
        }
        maximum = fmaxf(maximum, __shfl_xor(maximum, 32));
        bad |= __shfl_xor(bad, 32);
        const float scale = maximum / 127.0f;
        if (row >= mrows) continue;
        if (fc == 0 && (bad || (maximum > 0.0f && scale == 0.0f))) raise_error(S.err, kErrNumerical);
        const size_t prow = routed ? (size_t)(base + r0 + row) : (size_t)(r0 + row);
        if (fc == 0) sbase[prow * nb + blk] = scale;
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          uint32_t w = 0;
#pragma unroll
          for (int j = 0; j < 4; j++) {
            int qv = 0;
            if (scale != 0.0f) qv = (int)fminf(fmaxf(rintf(h[4 * g4 + j] / scale), -127.0f), 127.0f);
            w |= ((uint32_t)(uint8_t)(int8_t)qv) << (8 * j);
          }
          *reinterpret_cast<uint32_t*>(qbase + prow * W + hcol0 + 8 * g4 + 4 * fc) = w;
        }
      }
    }
  } else {
    float* out = routed ? S.y : S.ys;
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
      const int row = 32 * tt + row_in;
      if (row >= mrows) continue;
      const size_t at = (size_t)(base + r0 + row) * L.H;
#pragma unroll
      for (int ft = 0; ft < NFT; ft++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int n = n0 + wcol + 32 * ft + 8 * (r >> 2) + 4 * fc + (r & 3);
          if (n < N) out[at + n] = acc[ft][tt][r];
        }
    }
  }
}

// Int8Matrix::quantize (src/cpu/quantized.rs:43-74) of `rows` FP32 rows of
// width K (a multiple of 32): one thread per 32-block; non-finite input or
// an underflowing scale raises Numerical. Rows [split, rows) use width K2
// and start at src2/dst2/sc2 (the shared expert's hidden rows).
__global__ void quantize_rows_kernel(const float* __restrict__ src, int rows, int K,
                                     int8_t* __restrict__ dst, float* __restrict__ sc,
                                     const float* __restrict__ src2, int rows2, int K2,
                                     int8_t* __restrict__ dst2, float* __restrict__ sc2,
                                     int* err) {
  const long long nb1 = (long long)rows * (K / kQBlock);
  const long long nb2 = (long long)rows2 * (K2 / kQBlock);
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nb1 + nb2) return;
  const float* v;
  int8_t* q;
  float* s;
  if (i < nb1) {
    v = src + i * kQBlock;
    q = dst + i * kQBlock;
    s = sc + i;
  } else {
    const long long j = i - nb1;
    v = src2 + j * kQBlock;
    q = dst2 + j * kQBlock;
    s = sc2 + j;
  }
  float vals[kQBlock];
#pragma unroll
  for (int k = 0; k < kQBlock; k += 4) {
    const float4 f = *reinterpret_cast<const float4*>(v + k);
    vals[k] = f.x;
    vals[k + 1] = f.y;
    vals[k + 2] = f.z;
    vals[k + 3] = f.w;
  }
  float maximum = 0.0f;
  bool bad = false;
#pragma unroll
  for (int k = 0; k < kQBlock; k++) {
    bad |= !isfinite(vals[k]);
    maximum = fmaxf(maximum, fabsf(vals[k]));
  }
  const float scale = maximum / 127.0f;
  if (bad || (maximum > 0.0f && scale == 0.0f)) raise_error(err, kErrNumerical);
  *s = scale;
  uint32_t packed[kQBlock / 4];
#pragma unroll
  for (int k = 0; k < kQBlock; k += 4) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int qv = 0;
      if (scale != 0.0f) qv = (int)fminf(fmaxf(rintf(vals[k + j] / scale), -127.0f), 127.0f);
      w |= ((uint32_t)(uint8_t)(int8_t)qv) << (8 * j);
    }
    packed[k / 4] = w;
  }
#pragma unroll
  for (int k = 0; k < kQBlock / 4; k += 4)
    *reinterpret_cast<uint4*>(q + 4 * k) = make_uint4(packed[k], packed[k + 1], packed[k + 2],
                                                      packed[k + 3]);
}

void launch_quantize_rows(const float* src, int rows, int K, int8_t* dst, float* sc,
                          const float* src2, int rows2, int K2, int8_t* dst2, float* sc2,
                          int* err, hipStream_t s) {
  const long long blocks = (long long)rows * (K / kQBlock) + (long long)rows2 * (K2 / kQBlock);
  if (blocks == 0) return;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s,
                     src, rows, K, dst, sc, src2, rows2, K2, dst2, sc2, err);
}

bool i8_supported(const DeviceLayer& L) { return L.H % 64 == 0 && L.I % 64 == 0 && L.S % 64 == 0; }

static unsigned i8_grid(const DeviceLayer& L, int tiles_bound, bool gateup) {
  const int n = gateup ? std::max(2 * L.I, 2 * L.S) : L.H;
  const long long items = (long long)tiles_bound * ((n + i8_tile_n(gateup) - 1) / i8_tile_n(gateup));
  return (unsigned)((items + kI8Xcds - 1) / kI8Xcds * kI8Xcds);
}

// The traced instantiations run when the forward records any block sums or
// hidden rows; the plain gate/up then leaves FP32 hidden rows for the
// trace and for quantize_rows_kernel, otherwise it writes them quantised.
bool i8_traced(const Scratch& S, int T) {
  return S.q8.gateup || S.q8.down || S.q8.hidden ||
         (T == 1 && (S.q8.s_gateup || S.q8.s_down || S.q8.s_hidden));
}

void launch_i8_gateup(const DeviceLayer& L, const Scratch& S, const I8Planes& P, int T,
                      int tiles_bound, hipStream_t s) {
  const bool trace = i8_traced(S, T);
  auto* kern = trace ? i8_group_kernel<true, true> : i8_group_kernel<true, false>;
  hipLaunchKernelGGL(kern,
                     dim3(i8_grid(L, tiles_bound, true)), dim3(kI8Threads),
                     kI8Stages * i8_stage(true), s, L, S, P, T);
}

void launch_i8_down(const DeviceLayer& L, const Scratch& S, const I8Planes& P, int T,
                    int tiles_bound, hipStream_t s) {
  const bool trace = i8_traced(S, T);
  auto* kern = trace ? i8_group_kernel<false, true> : i8_group_kernel<false, false>;
  hipLaunchKernelGGL(kern,
                     dim3(i8_grid(L, tiles_bound, false)), dim3(kI8Threads),
                     kI8Stages * i8_stage(false), s, L, S, P, T);
}

}  // namespace uocr
