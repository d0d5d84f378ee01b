// One-token (decode) expert engine for INT8 overlays (weight-only and
// W8A8; BF16 layers take the row-dot engine of decode_rows.hip): bound by
// the bytes of the active experts' weights and by the latency of the steps
// that depend on each other (router logits -> selection -> expert rows ->
// output). One launch, four kinds of workgroup by id:
//   logit     ceil(E/8) workgroups: 8 router logits (one wave), stored
//             into every routed workgroup's copy (all waves) and for the
//             combine workgroups, which take the routing weights from them
//   shared    S/32 workgroups: 32 hidden values of the shared expert (no
//             routing needed), then their share of its down projection
//   routed    K (I/32) workgroups: wait for their copy of the E logits,
//             select, 32 hidden values of the expert of their slot, then
//             their share of its down projection
//   combine   H/8 workgroups: wait for the logits, select, then read the
//             down partials of 8 output features, sum each expert's in
//             block order, and the ordered combine.
// A gate/up workgroup's 32 hidden values are one 32-block of the down
// projection's reduction: it multiplies them into that block's 32 columns
// of every output row (one contiguous run of the k-blocked down panel,
// [W/32][H][32]) and publishes one partial per output feature. Only the
// partials cross workgroups, once: no hidden value is re-read by another
// workgroup.
//
// Cross-workgroup data. The logits, for the routed workgroups: one copy
// (64 words of Scratch::part, the sentinel 0xffffffff between launches)
// per routed workgroup, written device-coherently by the logit workgroups
// (8 words each), polled by its routed workgroup until no word is the
// sentinel, and set back to the sentinel by it. The logits, for the
// combine workgroups: the logit workgroups store them device-coherently,
// wait for the stores, count themselves in one word; the last one sets
// one flag line per combine workgroup and zeroes the count; a combine
// workgroup polls its own line and zeroes it. The partials: a region of
// 4-byte values (Scratch::part), each written by
// exactly one gate/up workgroup and read by exactly one combine workgroup,
// that holds the sentinel 0xffffffff between launches. A producer stores
// its value device-coherently (a value with the sentinel's bits becomes
// the quiet NaN 0x7fc00000); the consumer polls one probe of its run (the
// last routed producer's first values) until it is no longer the
// sentinel, then reads all its values with device-coherent loads until
// none is the sentinel, then writes the sentinel back. The probe only
// paces the polling: what orders the data is the sentinel check. So no
// word is counted into by more than the 8 logit workgroups, the partials
// are in their launch-start state again when the launch ends (also under
// graph replay: nothing depends on a launch counter), and a consumer sees
// each value as soon as its store lands. Why this shape: an agent-scope
// release / acquire fence per wave (an L2 write-back or invalidate each)
// made a call take 160 us instead of 17, and hundreds of waves counting
// into and polling one word took 80 us (accesses to one line serialise
// where the XCDs meet). The routed workgroups used to compute all E
// logits themselves from the router in L2 (160 KiB per workgroup): they
// selected at 4.6 us, against 4.3 us polling their copy (INT8 14.9 ->
// 14.5 us per token, W8A8 15.5 -> 14.9 us). Workgroups wait
// only on workgroups with smaller ids (logit < gate/up < combine). The
// dispatcher starts a launch's workgroups in id order, so every workgroup
// waited on has started, and none of those waits itself on a later one;
// every wait is bounded (kSpinLimit polls) and raises Resource when the
// bound is hit, so a launch always ends.
//
// Weights are read with range-checked buffer loads (out-of-range chunks
// read as zero without a memory access), all issued before the first use.
//
// Arithmetic is that of Decoder::projection / feed_forward for one row
// (src/decoder/mod.rs:99-122): INT8 weight-only as
// q * x summed per 16-byte chunk (gate/up) or per 32-block (down) and scaled
// once by the block scale (the reference rounds w = q * scale first,
// src/cpu/quantized.rs:119-131); W8A8 for DynamicActivations (one row is
// always a single-row group, :103-104) with the row quantised per 32-block
// and exact i32 block sums (:155-236) — each down block's term is the
// reference's ((float)sum * ws) * xs, and the combine adds an expert's block
// terms in block order from -0.0, as the reference accumulates them.
// Routing is moe::route (src/decoder/moe.rs:7-30) on logits from
// ops::linear (src/cpu/ops.rs:9-59); the combine follows
// src/decoder/mod.rs:185-194 (shared first, then ascending expert id, a
// multiply then an add).
#include "common.hpp"
#include "moe_kernels.hpp"
#include "routing.hpp"
#include "logit_copies.hpp"
#include "rowdot.hpp"

namespace uocr {

namespace {

constexpr int kWide = 2048;     // widest reduction dimension (H, S)
constexpr int kNarrow = 1024;   // widest routed intermediate size (I)
constexpr int kMaxK = 8;        // most routed experts per token
constexpr int kUpWaves = 8;                 // waves of a workgroup
constexpr int kThreads = 64 * kUpWaves;
constexpr int kHidPerWg = kUpWaves * 4;     // hidden values per gate/up workgroup
constexpr int kLogitsPerWg = 8;             // router rows per logit workgroup
constexpr int kFeatPerWg = 8;               // output features per combine workgroup
// Partials of one launch: S/32 shared blocks + K I/32 routed blocks.
constexpr int kMaxParts = kWide / kQBlock + kMaxK * kNarrow / kQBlock;
static_assert((size_t)kMaxParts * kWide * 4 <= kDecodePartBytes, "partial region");
// Polls of a wait (each followed by a short sleep, ~0.1-0.3 us) before it
// gives up and raises Resource: far beyond any launch's own duration.
constexpr int kSpinLimit = 1 << 20;
constexpr int kLine = 16;         // sync words per 64-byte line
constexpr int kErrResource = 6;  // uocr_status Resource
constexpr uint32_t kSentinel = kSlotSentinel;
static_assert((size_t)kMaxParts * kWide <= kDecodeCopyWord, "partials before the logit copies");


// Row of w13 holding gate value k (up value k is 32 rows further).
__device__ __forceinline__ int gate_row(int k) { return (k >> 5) * 64 + (k & 31); }

__device__ __forceinline__ int clamp_group(int g, int n) { return g < 0 ? 0 : (g >= n ? n - 1 : g); }

// Group g's INT8 gate/up rows and their scales; its down matrix as k-blocked
// panels ([W/32][H][32]) and their scales block-major ([W/32][H]).
__device__ __forceinline__ const void* w13_of(const DeviceLayer& L, int g) {
  return L.q13 + L.w13_offset(g);
}
__device__ __forceinline__ const float* s13_of(const DeviceLayer& L, int g) {
  return L.s13 + L.s13_offset(g);
}
__device__ __forceinline__ const void* w2k_of(const DeviceLayer& L, int g) {
  return L.q2k + L.w2_offset(g);
}
__device__ __forceinline__ const float* s2k_of(const DeviceLayer& L, int g) {
  return L.s2k + L.s2_offset(g);
}

struct GateUpSmem {
  float xl[kWide];
  int8_t xq[kWide];
  float xs[kWide / kQBlock];
  float logits[64];
  float h[kHidPerWg];     // this workgroup's hidden block
  int8_t hq[kHidPerWg];   // W8A8: the block quantised
  float hs[1];            // W8A8: its scale
  unsigned long long mask;
};

struct CombineSmem {
  // [feature][partial], rows padded by four words: each row starts 16-byte
  // aligned and the eight features' 16-byte reads fall in 32 different
  // banks.
  __align__(16) float part[kFeatPerWg][kMaxParts + 4];
  float y[kMaxK + 1][kFeatPerWg];     // per expert (slot order), then the shared expert
  float pw[kMaxK];
  unsigned long long mask;
};

union DecodeSmem {
  GateUpSmem up;
  CombineSmem comb;
};

// Device-coherent store and load of one value that another workgroup reads.
__device__ __forceinline__ void shared_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float shared_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kCoherent = 16;  // buffer-load cache policy: sc1 (device coherent)

__device__ __forceinline__ void sync_store(int* w, int v) {
  __hip_atomic_store(w, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int sync_add(int* w) {
  return __hip_atomic_fetch_add(w, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup counts: ceil(E/8) logit, S/32 shared and K I/32 routed gate/up,
// H/8 combine; and the partials (one per gate/up workgroup).
struct DecodeGrid {
  int n_logit, n_shared, n_routed, n_comb;
  __host__ __device__ DecodeGrid(const DeviceLayer& L)
      : n_logit((L.E + kLogitsPerWg - 1) / kLogitsPerWg),
        n_shared(L.S / kHidPerWg),
        n_routed(L.K * (L.I / kHidPerWg)),
        n_comb(L.H / kFeatPerWg) {}
  __host__ __device__ int blocks() const { return n_logit + n_up() + n_comb; }
  __host__ __device__ int n_up() const { return n_shared + n_routed; }
};

// The sync words: line 0 the logit count, then one flag line per combine
// workgroup for the logits.
struct SyncMap {
  int* logit_count;
  int* route_flag;
  __device__ SyncMap(int* w) : logit_count(w), route_flag(w + kLine) {}
};

__device__ __forceinline__ int wait_bound(const Scratch& S) {
  return S.wait_limit >= 0 ? S.wait_limit : kSpinLimit;
}

// A waiting workgroup's wave: polls its own flag, then zeroes it for the
// next launch; the wave's later memory accesses stay behind the poll.
// Gives up after the wait bound (Resource raised; the caller's results are
// then not valid, and the forward reports the error).
// Returns the flag's value (0 when the wait gave up).
__device__ __forceinline__ int wait_flag(int* flag, const Scratch& S) {
  int* err = S.err;
  const int bound = wait_bound(S);
  int v = 0;
  for (int n = 0;; n++) {
    v = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (v) break;
    if (n >= bound) {
      if ((threadIdx.x & 63) == 0) raise_error(err, kErrResource);
      break;
    }
    __builtin_amdgcn_s_sleep(4);
  }
  if ((threadIdx.x & 63) == 0) sync_store(flag, 0);
  asm volatile("" ::: "memory");
  return v;
}

// The launch's timeline (uocr_moe_trace::decode_stamps): thread 0 of the
// workgroup records the device's real-time counter (100 MHz) as stamp i of
// its workgroup, in LDS; the workgroup's last step writes the recorded
// stamps to its row (a global store before a barrier would stall the
// barrier, so the timeline would time its own stores). ST: the
// instantiation launched only when a timeline is asked for (the others
// carry no trace of it).
__shared__ unsigned long long g_stamps[kDecodeStamps];
__shared__ unsigned g_stamp_mask;
template <bool ST>
__device__ __forceinline__ void stamp(const Scratch&, int i) {
  if constexpr (ST) {
    if (threadIdx.x == 0) {
      g_stamps[i] = __builtin_amdgcn_s_memrealtime();
      g_stamp_mask |= 1u << i;
    }
  }
}
template <bool ST>
__device__ __forceinline__ void flush_stamps(const Scratch& S) {
  if constexpr (ST) {
    if (threadIdx.x == 0)
      for (int i = 0; i < kDecodeStamps; i++)
        if ((g_stamp_mask >> i) & 1u) S.stamps[(size_t)blockIdx.x * kDecodeStamps + i] = g_stamps[i];
  }
}

// Sets flags[0 .. n) (stride kLine) with the 64 lanes of one wave to v.
__device__ __forceinline__ void set_flags(int* flags, int n, int lane, int v) {
  for (int j = lane; j < n; j += 64) sync_store(flags + j * kLine, v);
}

// The token's selection from the E logits the logit workgroups published
// (one wave, after its flag).
__device__ __forceinline__ WaveSel select_token(const DeviceLayer& L, const Scratch& S, int* flag,
                                                int lane) {
  wait_flag(flag, S);
  const float v = lane < L.E ? shared_load(S.logits + lane) : 0.0f;
  return route_wave_sel(v, L.E, L.K);
}

// Logit workgroup b: router rows 8b + q and 8b + q + 4 (q = lane / 16; BF16
// router, FP32 x; rows past E read as zero) dotted with x by wave 0; every
// wave then stores the 8 logits (rows below E) into its share of the
// routed workgroups' copies, and wave 0 stores them for the combine
// workgroups, then counts in.
template <int KH, bool ST>
__device__ void logit_role(const DeviceLayer& L, const Scratch& S, GateUpSmem& sm,
                           const SyncMap& M, const DecodeGrid& G, int b, int wave, int lane) {
  const int q = lane >> 4;
  const int ra = kLogitsPerWg * b + q, rb = ra + 4;
  stamp<ST>(S, 0);
  float r0 = 0.0f, r1 = 0.0f;
  if (wave == 0) {
    RowPair<kBF16, KH> R;
    issue_rows(R, L.router, nullptr, L.E, L.H, ra, rb);
    RowStage<KH> X;
    load_row(X, S.xn, L.H, lane);
    store_row(X, sm.xl, L.H, lane);  // read back by this wave only
    dot_rows(R, L.H, sm.xl, nullptr, nullptr, r0, r1);
    if ((lane & 15) == 0) {
      sm.logits[q] = r0;
      sm.logits[q + 4] = r1;
    }
  }
  __syncthreads();
  publish_logits(S.part, sm.logits, b, L.E, G.n_routed, wave, kUpWaves, lane);
  if (wave != 0) return;
  if ((lane & 15) == 0) {
    if (ra < L.E) shared_store(S.logits + ra, r0);
    if (rb < L.E) shared_store(S.logits + rb, r1);
  }
  stamp<ST>(S, 1);
  // Counted once the logits are stored; the last logit workgroup releases
  // every combine workgroup waiting for them.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  stamp<ST>(S, 2);
  int last = 0;
  if (lane == 0) last = sync_add(M.logit_count) == G.n_logit - 1;
  if (__builtin_amdgcn_readfirstlane(last)) {
    set_flags(M.route_flag, G.n_comb, lane, 1);
    if (lane == 0) sync_store(M.logit_count, 0);
  }
  stamp<ST>(S, 3);
}

// Block c of group g's down matrix for one 32-value hidden block: output
// features f = tid + 512 r (r < kF), each the block's 32 consecutive int8
// panel elements (two 16-byte loads), and its block scale.
template <int KIND, int KH>
struct DownBlock {
  static_assert(KIND != kBF16, "INT8 overlays only");
  static constexpr int kF = (KH + kThreads - 1) / kThreads;  // features per thread
  static constexpr int kV = 2;                                // 16-byte loads per feature
  u32x4 w[kF][kV];
  float s[kF];
};

template <int KIND, int KH>
__device__ __forceinline__ void issue_down_block(DownBlock<KIND, KH>& D, const DeviceLayer& L,
                                                 int g, int c) {
  using DB = DownBlock<KIND, KH>;
  const int W = L.width(g);
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w2k_of(L, g), (uint32_t)W * L.H);
#pragma unroll
  for (int r = 0; r < DB::kF; r++) {
    const int f = tid + kThreads * r;
    const uint32_t off = f < L.H ? ((uint32_t)c * L.H + f) * kQBlock : kOut;
#pragma unroll
    for (int v = 0; v < DB::kV; v++)
      D.w[r][v] = __builtin_amdgcn_raw_buffer_load_b128(wr, off + 16u * v, 0, 0);
  }
  const int nb = W / kQBlock;
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(s2k_of(L, g), (uint32_t)L.H * nb * 4u);
#pragma unroll
  for (int r = 0; r < DB::kF; r++) {
    const int f = tid + kThreads * r;
    D.s[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        sr, f < L.H ? ((uint32_t)c * L.H + f) * 4u : kOut, 0, 0));
  }
}

// The partial of every output feature for the hidden block in sm (h, or
// hq / hs for W8A8), stored as partial p of the launch: feature f at
// part[((f / 8) NP + p) 8 + f % 8] (each combine workgroup's values are one
// contiguous run). W8A8 also stores the block's exact i32 sums at
// trace[f * tstride] (null: none).
template <int KIND, int KH>
__device__ __forceinline__ void down_partial(const DownBlock<KIND, KH>& D, const DeviceLayer& L,
                                             const Scratch& S, const GateUpSmem& sm, int p, int np,
                                             int32_t* trace, int tstride) {
  using DB = DownBlock<KIND, KH>;
  const int tid = threadIdx.x;
  float hv[kHidPerWg];
  if constexpr (KIND != kW8A8) {
#pragma unroll
    for (int j = 0; j < kHidPerWg; j += 4) {
      const float4 v = *reinterpret_cast<const float4*>(sm.h + j);
      hv[j] = v.x;
      hv[j + 1] = v.y;
      hv[j + 2] = v.z;
      hv[j + 3] = v.w;
    }
  }
  int hq4[kHidPerWg / 4];
  if constexpr (KIND == kW8A8) {
#pragma unroll
    for (int j = 0; j < kHidPerWg / 4; j++) hq4[j] = reinterpret_cast<const int*>(sm.hq)[j];
  }
  uint32_t* part = reinterpret_cast<uint32_t*>(S.part);
#pragma unroll
  for (int r = 0; r < DB::kF; r++) {
    const int f = tid + kThreads * r;
    if (f >= L.H) break;
    float y;
    if constexpr (KIND == kInt8) {
      // The block's 32 q * h products accumulate first (exact integers
      // times h), then one multiply by the block scale.
      float acc = 0.0f;
#pragma unroll
      for (int v = 0; v < DB::kV; v++)
#pragma unroll
        for (int i = 0; i < 16; i++)
          acc = fmaf((float)(int8_t)((D.w[r][v][i >> 2] >> (8 * (i & 3))) & 0xff), hv[16 * v + i],
                     acc);
      y = acc * D.s[r];
    } else {
      int sum = 0;
#pragma unroll
      for (int v = 0; v < DB::kV; v++)
#pragma unroll
        for (int i = 0; i < 4; i++) sum = __builtin_amdgcn_sdot4((int)D.w[r][v][i], hq4[4 * v + i], sum, false);
      if (trace) trace[(size_t)f * tstride] = sum;
      y = (float)sum * D.s[r] * sm.hs[0];
    }
    uint32_t bits = __float_as_uint(y);
    if (bits == kSentinel) bits = 0x7fc00000u;
    slot_store(part + ((size_t)(f / kFeatPerWg) * np + p) * kFeatPerWg + f % kFeatPerWg, bits);
  }
}

// After the gate/up dot: wave w's 16-lane group q holds hidden value
// 4 w + q of the block; into LDS, then quantised for W8A8. The FP32 row
// for a trace copy is stored after the partials (finish_block): a global
// store ahead of a barrier would hold the barrier until it completes (the
// barrier's workgroup release waits for the wave's stores).
template <int KIND>
__device__ __forceinline__ float hidden_block(const Scratch& S, GateUpSmem& sm, float r0, float r1,
                                              int wave, int lane) {
  const int kl = 4 * wave + (lane >> 4);
  const float h = silu(r0) * r1;
  if ((lane & 15) == 0) sm.h[kl] = h;
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    if (wave == 0) quantize_lds(sm.h, kHidPerWg, sm.hq, sm.hs, lane, S.err);
    __syncthreads();
  }
  return h;
}
__device__ __forceinline__ void finish_block(float* row, float h, int wave, int lane) {
  if ((lane & 15) == 0) row[4 * wave + (lane >> 4)] = h;
}

// Gate/up workgroup b. b < S/32: shared-expert hidden values 32b .. 32b+31
// (4 per wave: its 4 gate rows and the 4 matching up rows), h = silu(gate)
// * up, then partial b (shared down block b). After that: routed slot s =
// b' / (I/32), hidden values 32 c .. (c = b' % (I/32)) of the slot's expert,
// then partial S/32 + s I/32 + c (the expert's down block c); the first
// routed workgroup also writes the routing and the one-token dispatch (ids,
// weights, offsets, permutation, row tiles). The FP32 hidden row goes to
// gu (routed [K, I] in ascending slot, then shared [S]) for the W8A8 trace.
template <int KIND, int KH, bool ST>
__device__ void gateup_role(const DeviceLayer& L, const Scratch& S, GateUpSmem& sm,
                            const DecodeGrid& G, int b, int wave, int lane) {
  const int q = lane >> 4;
  const int n_shared = L.S / kHidPerWg;
  const int per_expert = L.I / kHidPerWg;
  const int np = G.n_up();
  // The down block: issued once the gate/up rows are dotted, except in a
  // routed W8A8 workgroup (issued behind the rows; see there). Issued with
  // the rows, it took HBM from them (the routed rows are on the critical
  // path: selection to rows dotted 3.4 -> 4.4 us, INT8).
  DownBlock<KIND, KH> D;
  stamp<ST>(S, 0);
  if (b < n_shared) {
    const int k = b * kHidPerWg + 4 * wave + q;
    const int ra = gate_row(k);
    // x first, so that staging it waits for x alone.
    RowStage<KH> X;
    if (wave == 0) load_row(X, S.xn, L.H, lane);
    RowPair<KIND, KH> P;
    issue_rows(P, w13_of(L, L.E), s13_of(L, L.E), 2 * L.S, L.H, ra, ra + 32);
    if (wave == 0) store_row(X, sm.xl, L.H, lane);
    __syncthreads();
    if constexpr (KIND == kW8A8) {
      quantize_lds_waves(sm.xl, L.H, sm.xq, sm.xs, wave, kUpWaves, lane, S.err);
      __syncthreads();
    }
    BlockSumOut bs;
    if (KIND == kW8A8 && S.q8.s_gateup) {
      const int nb = L.H / kQBlock;
      bs.a = S.q8.s_gateup + (size_t)k * nb;
      bs.b = S.q8.s_gateup + (size_t)(L.S + k) * nb;
      bs.na = bs.nb = nb;
    }
    float r0, r1;
    dot_rows(P, L.H, sm.xl, sm.xq, sm.xs, r0, r1, bs);
    issue_down_block(D, L, L.E, b);
    stamp<ST>(S, 3);
    const float h = hidden_block<KIND>(S, sm, r0, r1, wave, lane);
    int32_t* tr = KIND == kW8A8 && S.q8.s_down ? S.q8.s_down + b : nullptr;
    down_partial(D, L, S, sm, b, np, tr, L.S / kQBlock);
    finish_block(S.gu + (size_t)L.K * L.I + (size_t)b * kHidPerWg, h, wave, lane);
    stamp<ST>(S, 4);
    return;
  }
  const int rb = b - n_shared;
  const int slot = rb / per_expert;
  const int c = rb - slot * per_expert;
  // Wave 1 stages x while wave 0 polls this workgroup's copy of the logits
  // (set back to the sentinel at the end of the role).
  if (wave == 1) {
    RowStage<KH> X;
    load_row(X, S.xn, L.H, lane);
    store_row(X, sm.xl, L.H, lane);
  }
  if (wave == 0) sm.logits[lane] = poll_logits(S.part, rb, L.E, wait_bound(S), S.err, lane);
  __syncthreads();
  stamp<ST>(S, 1);
  // Wave 0 selects the token's experts for the workgroup.
  if (wave == 0) {
    const WaveSel r = route_wave_sel(sm.logits[lane], L.E, L.K);
    if (lane == 0) sm.mask = r.mask;
  }
  __syncthreads();
  stamp<ST>(S, 2);
  const int g = clamp_group(__builtin_amdgcn_readfirstlane(slot_expert(sm.mask, slot)), L.E);
  const int k = kHidPerWg * c + 4 * wave + q;
  const int ra = gate_row(k);
  RowPair<KIND, KH> P;
  issue_rows(P, w13_of(L, g), s13_of(L, g), 2 * L.I, L.H, ra, ra + 32);
  // W8A8: x quantised per 32-block while the rows are in flight (the
  // barrier waits for LDS traffic only), and the down block issued behind
  // them: its dot (v_dot4 block sums) is slower than the weight-only one,
  // and with the block in flight during it the token took 14.75 against
  // 15.1 us. Weight-only issues the block after the dot (issued here, it
  // took HBM from the gate/up rows: 14.5 -> 15.1 us).
  if constexpr (KIND == kW8A8) {
    quantize_lds_waves(sm.xl, L.H, sm.xq, sm.xs, wave, kUpWaves, lane, S.err);
    __syncthreads();
    issue_down_block(D, L, g, c);
  }
  // One token: the dispatched position of a slot is the slot itself.
  BlockSumOut bs;
  if (KIND == kW8A8 && S.q8.gateup) {
    const int nb = L.H / kQBlock;
    bs.a = S.q8.gateup + ((size_t)slot * 2 * L.I + k) * nb;
    bs.b = S.q8.gateup + ((size_t)slot * 2 * L.I + L.I + k) * nb;
    bs.na = bs.nb = nb;
  }
  float r0, r1;
  dot_rows(P, L.H, sm.xl, sm.xq, sm.xs, r0, r1, bs);
  if constexpr (KIND != kW8A8) issue_down_block(D, L, g, c);
  stamp<ST>(S, 3);
  const float h = hidden_block<KIND>(S, sm, r0, r1, wave, lane);
  const int nbI = L.I / kQBlock;
  int32_t* tr = KIND == kW8A8 && S.q8.down ? S.q8.down + (size_t)slot * L.H * nbI + c : nullptr;
  down_partial(D, L, S, sm, b, np, tr, nbI);
  finish_block(S.gu + (size_t)slot * L.I + (size_t)c * kHidPerWg, h, wave, lane);
  if (wave == 0) release_logits(S.part, rb, L.E, lane);
  // The first routed workgroup writes the routing and the one-token
  // dispatch last (its stores are off the path to the partials).
  if (rb == 0 && wave == 0) {
    const WaveSel r = route_wave_sel(sm.logits[lane], L.E, L.K);
    const float w = route_weight(r, L.normalize, L.scale);
    if (!r.ok && lane == 0) raise_error(S.err, kErrNumerical);
    const unsigned long long below_mask = r.mask & ((1ull << lane) - 1ull);
    const int asc = __popcll(below_mask);  // ascending slot / selected ids below lane
    if ((r.mask >> lane) & 1ull) {
      S.topk_ids[r.rank] = lane;
      S.topk_w[r.rank] = w;
      S.inv_pos[r.rank] = asc;
      S.perm_rows[asc] = 0;
      S.perm_w[asc] = w;
      S.tiles[2 * asc] = lane;
      S.tiles[2 * asc + 1] = 0;
    }
    if (lane < L.E) S.offsets[lane] = asc;
    if (lane == 0) {
      S.offsets[L.E] = L.K;
      S.tiles[2 * L.K] = L.E;
      S.tiles[2 * L.K + 1] = 0;
      S.counters[0] = L.K + 1;
      S.counters[1] = L.K;
      S.counters[2] = L.K;
      S.counters[3] = L.K;
    }
  }
  stamp<ST>(S, 4);
}

// Combine workgroup b: output features 8b .. 8b+7. Wave 0 waits for the
// logits and selects (the routing weights in ascending slot order), then
// polls one probe of its run (the last routed producer's first four
// values: the routed producers finish together, after the shared ones)
// until it is no longer the sentinel; the workgroup then reads its NP x 8
// partials (a contiguous run, a line no other workgroup polls) until none
// is the sentinel, writes the sentinel back, sums each expert's blocks in
// block order (each slot's, then the shared expert's) and combines:
// out = (residual +) (y_shared + p_0 y_0 + p_1 y_1 + ...), mul then add.
template <int KIND, bool ST>
__device__ void combine_role(const DeviceLayer& L, const Scratch& S, CombineSmem& sm,
                             const SyncMap& M, const DecodeGrid& G, int b, const float* residual,
                             float* out, int wave, int lane) {
  const int tid = threadIdx.x;
  const int f0 = kFeatPerWg * b;
  const int np = G.n_up();
  const int bound = wait_bound(S);
  stamp<ST>(S, 0);
  if (wave == 0) {
    const WaveSel r = select_token(L, S, M.route_flag + b * kLine, lane);
    const float w = route_weight(r, L.normalize, L.scale);
    const int asc = __popcll(r.mask & ((1ull << lane) - 1ull));
    if ((r.mask >> lane) & 1ull) sm.pw[asc] = w;
    if (lane == 0) sm.mask = r.mask;
    stamp<ST>(S, 1);
  }
  // NP x 8 floats = 2 NP float4, thread tid takes float4 tid + 512 m.
  constexpr int kM = (2 * kMaxParts + kThreads - 1) / kThreads;
  const int n4 = 2 * np;
  uint32_t* run = reinterpret_cast<uint32_t*>(S.part) + (size_t)b * np * kFeatPerWg;
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(run, (uint32_t)n4 * 16u);
  if (wave == 0) {
    // The probe: a hint only (the data wait below checks every value).
    for (int it = 0;; it++) {
      const u32x4 pv = __builtin_amdgcn_raw_buffer_load_b128(rr, (uint32_t)(n4 - 2) * 16u, 0,
                                                             kCoherent);
      if (pv.x != kSentinel && pv.y != kSentinel && pv.z != kSentinel && pv.w != kSentinel) break;
      if (it >= bound) break;  // the data wait below raises the error
      __builtin_amdgcn_s_sleep(4);
    }
  }
  __syncthreads();
  stamp<ST>(S, 2);
  const float res_f = residual && tid < kFeatPerWg ? residual[f0 + tid] : 0.0f;
  u32x4 v[kM];
  bool pend[kM];
#pragma unroll
  for (int m = 0; m < kM; m++) {
    v[m] = u32x4{0u, 0u, 0u, 0u};
    pend[m] = tid + kThreads * m < n4;
  }
  for (int it = 0;; it++) {
    bool any = false;
#pragma unroll
    for (int m = 0; m < kM; m++) {
      if (pend[m]) {
        v[m] = __builtin_amdgcn_raw_buffer_load_b128(rr, (uint32_t)(tid + kThreads * m) * 16u, 0,
                                                     kCoherent);
        pend[m] = v[m].x == kSentinel || v[m].y == kSentinel || v[m].z == kSentinel ||
                  v[m].w == kSentinel;
        any |= pend[m];
      }
    }
    if (!__syncthreads_or(any)) break;
    if (it >= bound) {
      if (tid == 0) raise_error(S.err, kErrResource);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  stamp<ST>(S, 3);
  // Into LDS feature-major ([feature][partial]).
#pragma unroll
  for (int m = 0; m < kM; m++) {
    const int i = tid + kThreads * m;
    if (i < n4) {
      const int p = i >> 1, j0 = (i & 1) * 4;
      sm.part[j0][p] = __uint_as_float(v[m].x);
      sm.part[j0 + 1][p] = __uint_as_float(v[m].y);
      sm.part[j0 + 2][p] = __uint_as_float(v[m].z);
      sm.part[j0 + 3][p] = __uint_as_float(v[m].w);
    }
  }
  __syncthreads();
  // Per expert and feature, its blocks in order from -0.0 (Rust's float
  // sum): wave 0 lane 8 s + j slot s < K (partials S/32 + s I/32 ..), wave
  // 1 lane j the shared expert (partials 0 .. S/32). The block count and the
  // row alignment are wave-uniform, so the loops branch on scalars.
  const int n_shared = L.S / kHidPerWg, per_expert = L.I / kHidPerWg;
  if (wave < 2) {
    const bool shared = wave == 1;
    const int e = shared ? L.K : lane / kFeatPerWg, j = lane % kFeatPerWg;
    const int nb = __builtin_amdgcn_readfirstlane(shared ? n_shared : per_expert);
    const int p0 = shared ? 0 : n_shared + e * per_expert;
    const bool active = shared ? lane < kFeatPerWg : lane < L.K * kFeatPerWg;
    const float* row = &sm.part[j][active ? p0 : 0];
    float acc = -0.0f;
    if (((n_shared | per_expert) & 3) == 0) {
      // 16-byte reads (rows and p0 16-byte aligned), all issued before the
      // adds.
      constexpr int kMaxQuads = kWide / kQBlock / 4;  // S/32 <= 64 blocks
      const float4* quad = reinterpret_cast<const float4*>(row);
      const int nq = nb / 4;
      float4 t[kMaxQuads];
#pragma unroll
      for (int u = 0; u < kMaxQuads; u++)
        if (u < nq) t[u] = quad[u];
#pragma unroll
      for (int u = 0; u < kMaxQuads; u++) {
        if (u < nq) {
          acc += t[u].x;
          acc += t[u].y;
          acc += t[u].z;
          acc += t[u].w;
        }
      }
    } else {
      for (int i = 0; i < nb; i++) acc += row[i];
    }
    if (active) sm.y[e][j] = acc;
  }
  __syncthreads();
  stamp<ST>(S, 4);
  if (tid < kFeatPerWg) {
    float acc = sm.y[L.K][tid];
#pragma unroll
    for (int s = 0; s < kMaxK; s++)
      if (s < L.K) acc = acc + sm.pw[s] * sm.y[s][tid];
    if (residual) acc = res_f + acc;
    out[f0 + tid] = acc;
  }
  // The sentinel back into every value read, after the last barrier (a
  // global store ahead of a barrier would hold it until the store lands).
  const u32x4 sent = {kSentinel, kSentinel, kSentinel, kSentinel};
#pragma unroll
  for (int m = 0; m < kM; m++) {
    const int i = tid + kThreads * m;
    if (i < n4) __builtin_amdgcn_raw_buffer_store_b128(sent, rr, (uint32_t)i * 16u, 0, kCoherent);
  }
  stamp<ST>(S, 5);
}

template <int KIND, int KH, bool ST>
__global__ __launch_bounds__(kThreads) void decode_kernel(DeviceLayer L, Scratch S,
                                                          const float* residual, float* out) {
  __shared__ __align__(16) DecodeSmem sm;
  // Wave-uniform (scalar) so the per-wave buffer bases stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const DecodeGrid G(L);
  const SyncMap M(S.sync);
  if constexpr (ST) {
    if (threadIdx.x == 0) g_stamp_mask = 0;
  }
  int b = blockIdx.x;
  if (b < G.n_logit) {
    logit_role<KH, ST>(L, S, sm.up, M, G, b, wave, lane);
  } else if ((b -= G.n_logit) < G.n_up()) {
    gateup_role<KIND, KH, ST>(L, S, sm.up, G, b, wave, lane);
  } else {
    b -= G.n_up();
    combine_role<KIND, ST>(L, S, sm.comb, M, G, b, residual, out, wave, lane);
  }
  flush_stamps<ST>(S);
}

template <int KIND, int KH>
void launch_kind(const DeviceLayer& L, const Scratch& S, const float* residual, float* out,
                 hipStream_t s) {
  const DecodeGrid G(L);
  if (S.stamps)
    decode_kernel<KIND, KH, true><<<dim3(G.blocks()), dim3(kThreads), 0, s>>>(L, S, residual, out);
  else
    decode_kernel<KIND, KH, false><<<dim3(G.blocks()), dim3(kThreads), 0, s>>>(L, S, residual, out);
}

template <int KH>
void launch_width(const DeviceLayer& L, const Scratch& S, const float* residual, float* out,
                  hipStream_t s) {
  if (L.quant_mode == 1)
    launch_kind<kInt8, KH>(L, S, residual, out, s);
  else
    launch_kind<kW8A8, KH>(L, S, residual, out, s);
}

}  // namespace

bool splitk_decode_supported(const DeviceLayer& L) {
  // Gate/up rows reduce over H (<= 2048), 32 hidden values per workgroup,
  // each a 32-block of the down projection's reduction; the combine takes 8
  // output features per workgroup; routing is one wave over E <= 64 logits.
  // The sync words: the logit count line and a flag line per combine
  // workgroup (H/8 <= 256) fit kDecodeSyncBytes; the partials (S/32 + K
  // I/32 per feature) fit kDecodePartBytes.
  static_assert((1 + kWide / kFeatPerWg) * kLine * 4 <= (int)kRouterSyncWord * 4,
                "decode sync words before the router's");
  static_assert(kLogitsPerWg == 8 && kHidPerWg == 32 && kFeatPerWg == 8,
                "the timeline's row count (UOCR_DECODE_STAMP_ROWS) follows these widths");
  return L.H <= kWide && L.S <= kWide && L.I <= kNarrow && L.K >= 1 && L.K <= kMaxK &&
         L.E <= 64 && L.H % kFeatPerWg == 0 && L.I % kHidPerWg == 0 && L.S % kHidPerWg == 0;
}

bool decode_supported(const DeviceLayer& L) {
  return L.quant_mode == 0 ? rows_decode_supported(L) : splitk_decode_supported(L);
}

void launch_decode(const DeviceLayer& L, const Scratch& S, const float* residual, float* out,
                   hipStream_t s) {
  if (L.quant_mode == 0)
    launch_rows_decode(L, S, residual, out, s);
  else if (L.H <= 1280)
    launch_width<1280>(L, S, residual, out, s);
  else
    launch_width<kWide>(L, S, residual, out, s);
}

}  // namespace uocr
