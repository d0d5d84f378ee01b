// One-token (decode) expert engine for BF16 layers (INT8 overlays take the
// split-K engine of decode.hip, whose down blocks are half as many bytes):
// bound by the bytes of the active experts' weights and by the latency of
// the steps that depend on each other (router logits -> selection -> expert
// rows; hidden values -> down). Here the down rows stream on workgroups of
// their own while the hidden values are handed over, which hides the
// 13.8 MB of routed BF16 down rows that the split-K engine would load after
// the gate/up dot (17.8 against 19.4 us per token).
// One launch, four kinds of workgroup by id:
//   logit     ceil(E/8) workgroups, one wave each: 8 router logits
//   shared    S/32 workgroups: shared-expert gate/up (no routing needed)
//   routed    K (I/32) workgroups: all E router logits (from L2: the
//             router is 160 KiB), select, gate/up of the expert of their
//             slot (routing in the workgroup is ~2 us sooner than waiting
//             for the logit workgroups)
//   down      H/8 workgroups: wait for the logits, select, issue the down
//             rows of every selected expert, wait for every gate/up wave,
//             then the routed and shared down of 8 output features and
//             their ordered combine.
// Workgroups wait only on workgroups with smaller ids (logit < gate/up <
// down). The dispatcher starts a launch's workgroups in id order, so every
// workgroup waited on has started, and none of those waits itself on a
// later one; every wait is also bounded (kSpinLimit polls) and raises
// Resource when the bound is hit, so a launch always ends.
//
// Cross-workgroup words (Scratch::sync, kDecodeSyncBytes, zero before the
// launch; 64-byte lines): a count of logit workgroups done, 16 sub-counts
// of gate/up workgroups done (gate/up workgroup b counts in sub-count b %
// 16), one flag line per workgroup waiting for the logits and one line of
// 16 flags per down workgroup (flag i: sub-set i of the gate/up
// workgroups is done). The data that crosses workgroups (the logits, the
// hidden rows) is written and read only with device-coherent accesses
// (sc1: agent-scope relaxed atomic stores and loads, sc1 buffer loads),
// which neither leave it in nor read it from a cache that another XCD's
// writes bypass. A producer waits for its stores to complete (vmcnt 0)
// before it counts itself; the workgroup whose count completes a set sets
// the flag of every workgroup waiting for that set and zeroes the count;
// a waiting workgroup polls its own line, zeroes it, then reads the data.
// So every word is zero again when the launch ends. Why this shape: an
// agent-scope release / acquire fence per wave (an L2 write-back or
// invalidate each) made a call take 160 us instead of 17, and hundreds of
// waves counting into and polling one word took 80 us (accesses to one
// line serialise where the XCDs meet); now every poll has a line of its
// own and at most 14 workgroups count into one word.
//
// Weights are read with range-checked buffer loads (out-of-range chunks
// read as zero without a memory access), all issued before the first use.
//
// Arithmetic is that of Decoder::projection / feed_forward for one row
// (src/decoder/mod.rs:99-122): BF16 weights widened exactly. Routing is moe::route (src/decoder/moe.rs:7-30) on logits from
// ops::linear (src/cpu/ops.rs:9-59); the combine follows src/decoder/mod.rs:185-194.
#include "common.hpp"
#include "moe_kernels.hpp"
#include "routing.hpp"
#include "rowdot.hpp"

namespace uocr {

namespace {

constexpr int kWide = 2048;     // widest reduction dimension (H, S)
constexpr int kNarrow = 1024;   // widest routed intermediate size (I)
constexpr int kMaxK = 8;        // most routed experts per token
constexpr int kUpWaves = 8;                 // waves of a gate/up workgroup
constexpr int kHidPerWg = kUpWaves * 4;     // hidden values per gate/up workgroup
constexpr int kLogitsPerWg = 8;             // router rows per logit workgroup
// Polls of a wait (each followed by a short sleep, ~0.1 us) before it gives
// up and raises Resource: far beyond any launch's own duration.
constexpr int kSpinLimit = 1 << 20;
constexpr int kLine = 16;         // sync words per 64-byte line
constexpr int kSubCounts = 16;    // gate/up sub-counts
constexpr int kErrResource = 6;  // uocr_status Resource

// Row of w13 holding gate value k (up value k is 32 rows further).
__device__ __forceinline__ int gate_row(int k) { return (k >> 5) * 64 + (k & 31); }

__device__ __forceinline__ int clamp_group(int g, int n) { return g < 0 ? 0 : (g >= n ? n - 1 : g); }

__device__ __forceinline__ const void* w13_of(const DeviceLayer& L, int g) {
  return L.w13 + L.w13_offset(g);
}
__device__ __forceinline__ const void* w2_of(const DeviceLayer& L, int g) {
  return L.w2 + L.w2_offset(g);
}

struct GateUpSmem {
  float xl[kWide];
  float logits[64];
  unsigned long long mask;
};

struct DownSmem {
  float hl[kMaxK + 2][kNarrow];
  float yl[kMaxK + 2][8];
  float pw[kMaxK];
  unsigned long long mask;
};

union DecodeSmem {
  GateUpSmem up;
  DownSmem down;
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
// H/8 down.
struct DecodeGrid {
  int n_logit, n_shared, n_routed, n_down;
  __host__ __device__ DecodeGrid(const DeviceLayer& L)
      : n_logit((L.E + kLogitsPerWg - 1) / kLogitsPerWg),
        n_shared(L.S / kHidPerWg),
        n_routed(L.K * (L.I / kHidPerWg)),
        n_down(L.H / 8) {}
  __host__ __device__ int blocks() const { return n_logit + n_shared + n_routed + n_down; }
  __host__ __device__ int n_up() const { return n_shared + n_routed; }
};

// The sync words: line 0 the logit count, lines 1..16 the gate/up
// sub-counts, then one flag line per down workgroup for the logits and one
// line of sub-set flags per down workgroup.
struct SyncMap {
  int* logit_count;
  int* sub;
  int* route_flag;
  int* down_flags;
  __device__ SyncMap(int* w, const DecodeGrid& G)
      : logit_count(w),
        sub(w + kLine),
        route_flag(w + (1 + kSubCounts) * kLine),
        down_flags(w + (1 + kSubCounts + G.n_down) * kLine) {}
};

// A waiting workgroup's wave: polls its own flag, then zeroes it for the
// next launch; the wave's later memory accesses stay behind the poll.
// Gives up after kSpinLimit polls (Resource raised; the caller's results
// are then not valid, and the forward reports the error).
__device__ __forceinline__ int wait_bound(const Scratch& S) {
  return S.wait_limit >= 0 ? S.wait_limit : kSpinLimit;
}
__device__ __forceinline__ void wait_flag(int* flag, const Scratch& S) {
  int* err = S.err;
  const int bound = wait_bound(S);
  for (int n = 0;; n++) {
    const int v = __builtin_amdgcn_readfirstlane(
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
}

// The launch's timeline (uocr_moe_trace::decode_stamps): thread 0 of the
// workgroup stores the device's real-time counter (100 MHz) as stamp i of
// its workgroup's row. ST: the instantiation launched only when a timeline
// is asked for (the others carry no trace of it).
template <bool ST>
__device__ __forceinline__ void stamp(const Scratch& S, int i) {
  if constexpr (ST) {
    if (threadIdx.x == 0)
      S.stamps[(size_t)blockIdx.x * kDecodeStamps + i] = __builtin_amdgcn_s_memrealtime();
  }
}

// Sets flags[0 .. n) (stride kLine) with the 64 lanes of one wave.
__device__ __forceinline__ void set_flags(int* flags, int n, int lane) {
  for (int j = lane; j < n; j += 64) sync_store(flags + j * kLine, 1);
}

// The token's selection from the E logits the logit workgroups published
// (one wave, after its flag).
__device__ __forceinline__ WaveSel select_token(const DeviceLayer& L, const Scratch& S, int* flag,
                                                int lane) {
  wait_flag(flag, S);
  const float v = lane < L.E ? shared_load(S.logits + lane) : 0.0f;
  return route_wave_sel(v, L.E, L.K);
}

// End of a gate/up workgroup (every wave calls it once its hidden values
// are stored): counts the workgroup in sub-count b % 16; the one completing
// its sub-set sets that sub-set's flag in every down workgroup's line and
// zeroes the sub-count.
__device__ __forceinline__ void count_gateup(const SyncMap& M, const DecodeGrid& G, int b, int wave,
                                             int lane) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's stores are complete
  __syncthreads();
  if (wave != 0) return;
  const int i = b % kSubCounts;
  int last = 0;
  if (lane == 0) last = sync_add(M.sub + i * kLine) == (G.n_up() - 1 - i) / kSubCounts;
  if (__builtin_amdgcn_readfirstlane(last)) {
    for (int j = lane; j < G.n_down; j += 64) sync_store(M.down_flags + j * kLine + i, 1);
    if (lane == 0) sync_store(M.sub + i * kLine, 0);
  }
}

// A down workgroup's wave 0: polls its line until the flags of all n
// gate/up sub-sets are set, then zeroes them (bounded like wait_flag).
__device__ __forceinline__ void wait_line(int* line, int n, const Scratch& S) {
  int* err = S.err;
  const int bound = wait_bound(S);
  const int lane = threadIdx.x & 63;
  const unsigned long long want = (1ull << n) - 1ull;
  for (int it = 0;; it++) {
    const int v = lane < n ? __hip_atomic_load(line + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    if ((__ballot(v != 0) & want) == want) break;
    if (it >= bound) {
      if (lane == 0) raise_error(err, kErrResource);
      break;
    }
    __builtin_amdgcn_s_sleep(4);
  }
  if (lane < n) sync_store(line + lane, 0);
  asm volatile("" ::: "memory");
}

// Stages the activation row (wave 0) into LDS; the caller's loads stay in
// flight meanwhile.
template <int KH>
__device__ __forceinline__ void stage_x(const DeviceLayer& L, const Scratch& S, GateUpSmem& sm,
                                        int wave, int lane) {
  if (wave == 0) {
    RowStage<KH> X;
    load_row(X, S.xn, L.H, lane);
    store_row(X, sm.xl, L.H, lane);
  }
  __syncthreads();
}

// Logit workgroup b: router rows 8b + q and 8b + q + 4 (q = lane / 16; BF16
// router, FP32 x; rows past E read as zero) dotted with x by one wave.
template <int KH, bool ST>
__device__ void logit_role(const DeviceLayer& L, const Scratch& S, GateUpSmem& sm,
                           const SyncMap& M, const DecodeGrid& G, int b, int lane) {
  const int q = lane >> 4;
  const int ra = kLogitsPerWg * b + q, rb = ra + 4;
  stamp<ST>(S, 0);
  RowPair<kBF16, KH> R;
  issue_rows(R, L.router, nullptr, L.E, L.H, ra, rb);
  RowStage<KH> X;
  load_row(X, S.xn, L.H, lane);
  store_row(X, sm.xl, L.H, lane);  // read back by this wave only
  float r0, r1;
  dot_rows(R, L.H, sm.xl, nullptr, nullptr, r0, r1);
  if ((lane & 15) == 0) {
    if (ra < L.E) shared_store(S.logits + ra, r0);
    if (rb < L.E) shared_store(S.logits + rb, r1);
  }
  stamp<ST>(S, 1);
  // Counted once the logits are stored; the last logit workgroup releases
  // every workgroup waiting for them.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  stamp<ST>(S, 2);
  int last = 0;
  if (lane == 0) last = sync_add(M.logit_count) == G.n_logit - 1;
  if (__builtin_amdgcn_readfirstlane(last)) {
    set_flags(M.route_flag, G.n_down, lane);
    if (lane == 0) sync_store(M.logit_count, 0);
  }
  stamp<ST>(S, 3);
}

// Gate/up workgroup b. b < S/32: shared-expert hidden values 32b .. 32b+31
// (4 per wave: its 4 gate rows and the 4 matching up rows), h = silu(gate)
// * up into gu[K*I ..]. After that: routed slot s = b' / (I/32), hidden
// values 32 (b' % (I/32)) .., into gu[s * I ..]; the first routed workgroup
// also writes the routing and the one-token dispatch (ids, weights,
// offsets, permutation, row tiles). Each wave counts itself done once its
// hidden values are stored.
template <int KH, bool ST>
__device__ void gateup_role(const DeviceLayer& L, const Scratch& S, GateUpSmem& sm,
                            const SyncMap& M, const DecodeGrid& G, int b, int wave, int lane) {
  const int q = lane >> 4;
  const int n_shared = L.S / kHidPerWg;
  const int per_expert = L.I / kHidPerWg;
  stamp<ST>(S, 0);
  if (b < n_shared) {
    const int k = b * kHidPerWg + 4 * wave + q;
    const int ra = gate_row(k);
    RowPair<kBF16, KH> P;
    issue_rows(P, w13_of(L, L.E), nullptr, 2 * L.S, L.H, ra, ra + 32);
    stage_x<KH>(L, S, sm, wave, lane);
    float r0, r1;
    dot_rows(P, L.H, sm.xl, nullptr, nullptr, r0, r1);
    stamp<ST>(S, 3);
    if ((lane & 15) == 0) shared_store(S.gu + (size_t)L.K * L.I + k, silu(r0) * r1);
    count_gateup(M, G, b, wave, lane);
    stamp<ST>(S, 4);
    return;
  }
  const int rb = b - n_shared;
  const int slot = rb / per_expert;
  // Router rows 8 wave + q and 8 wave + q + 4 (BF16 router, FP32 x; rows
  // past E read as zero), the logits into LDS; x is issued first, so it is
  // staged while the router rows are still in flight. Same rows and the
  // same dot as the logit workgroups: the same logits, bit for bit.
  {
    RowStage<KH> X;
    if (wave == 0) load_row(X, S.xn, L.H, lane);
    RowPair<kBF16, KH> R;
    issue_rows(R, L.router, nullptr, L.E, L.H, 8 * wave + q, 8 * wave + q + 4);
    if (wave == 0) store_row(X, sm.xl, L.H, lane);
    __syncthreads();
    stamp<ST>(S, 1);
    float r0, r1;
    dot_rows(R, L.H, sm.xl, nullptr, nullptr, r0, r1);
    if ((lane & 15) == 0) {
      sm.logits[8 * wave + q] = r0;
      sm.logits[8 * wave + q + 4] = r1;
    }
  }
  __syncthreads();
  // Wave 0 selects the token's experts and publishes the selection; the
  // first routed workgroup's wave 0 also writes the routing and the
  // one-token dispatch (ids, weights, offsets, permutation, row tiles).
  if (wave == 0) {
    const WaveSel r = route_wave_sel(sm.logits[lane], L.E, L.K);
    if (lane == 0) sm.mask = r.mask;
    if (rb == 0) {
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
  }
  __syncthreads();
  stamp<ST>(S, 2);
  const int g = clamp_group(__builtin_amdgcn_readfirstlane(slot_expert(sm.mask, slot)), L.E);
  const int k = kHidPerWg * (rb - slot * per_expert) + 4 * wave + q;
  const int ra = gate_row(k);
  RowPair<kBF16, KH> P;
  issue_rows(P, w13_of(L, g), nullptr, 2 * L.I, L.H, ra, ra + 32);
  float r0, r1;
  dot_rows(P, L.H, sm.xl, nullptr, nullptr, r0, r1);
  stamp<ST>(S, 3);
  if ((lane & 15) == 0) shared_store(S.gu + (size_t)slot * L.I + k, silu(r0) * r1);
  count_gateup(M, G, b, wave, lane);
  stamp<ST>(S, 4);
}

// Down workgroup b: output features 8b .. 8b+7; wave w < K = the selected
// expert of ascending slot w, waves K and K+1 = the two halves of the
// shared expert's reduction (S/2 columns each); then the ordered combine
// of the 8 features: out = (residual +) ((y_s0 + y_s1) + p_0 y_0 + p_1 y_1
// + ...), mul then add.
template <bool ST>
__device__ void down_role(const DeviceLayer& L, const Scratch& S, DownSmem& sm, const SyncMap& M,
                          const DecodeGrid& G, int b, const float* residual, float* out, int wave,
                          int lane) {
  const int q = lane >> 4;
  const int f0 = 8 * b;
  const bool routed = wave < L.K;
  const int half = L.S / 2;
  stamp<ST>(S, 0);
  // This wave's hidden row: an expert's I values, or half the shared S.
  const int n = routed ? L.I : half;
  // The shared expert's rows need no routing: issued first.
  RowPair<kBF16, kNarrow> P;
  if (!routed)
    issue_rows_cols(P, w2_of(L, L.E), nullptr, L.H, L.S, (wave - L.K) * half, n, f0 + q, f0 + q + 4);
  // Wave 0 selects; every routed wave needs its slot's expert, the combine
  // the routing weights in ascending slot order.
  if (wave == 0) {
    const WaveSel r = select_token(L, S, M.route_flag + b * kLine, lane);
    const float w = route_weight(r, L.normalize, L.scale);
    const int asc = __popcll(r.mask & ((1ull << lane) - 1ull));
    if ((r.mask >> lane) & 1ull) sm.pw[asc] = w;
    if (lane == 0) sm.mask = r.mask;
  }
  __syncthreads();
  stamp<ST>(S, 1);
  const int g =
      routed ? clamp_group(__builtin_amdgcn_readfirstlane(slot_expert(sm.mask, wave)), L.E) : L.E;
  if (routed) {
    // The routed down rows are needed only once every hidden value is in
    // (~6 us after the selection), while the routed gate/up rows, read from
    // HBM at the same time, are on the critical path: issued at once, they
    // took a third of HBM from them. They wait for the time those rows take
    // at the HBM peak (80 KB per 10 ns tick) less 0.44 us — 2.9 us at the
    // model shape, measured best of 1.0-5.0 us (per token 18.4 -> 17.9 us);
    // issuing them after the hidden values were in cost 0.8 us instead. A
    // wait on the real-time counter always ends.
    const long long up_bytes = (long long)L.K * 2 * L.I * L.H * 2;
    const long long ticks = up_bytes / 81920 - 44;
    if (ticks > 0) {
      const unsigned long long t_end = __builtin_amdgcn_s_memrealtime() + (unsigned long long)ticks;
      while (__builtin_amdgcn_s_memrealtime() < t_end) __builtin_amdgcn_s_sleep(2);
    }
    issue_rows_cols(P, w2_of(L, g), nullptr, L.H, L.I, 0, n, f0 + q, f0 + q + 4);
  }
  const float res_f = residual ? residual[f0 + (lane & 7)] : 0.0f;
  // The hidden rows are whole once every gate/up workgroup has counted
  // itself (wave 0 waits for this workgroup's flag).
  if (wave == 0) wait_line(M.down_flags + b * kLine, G.n_up() < kSubCounts ? G.n_up() : kSubCounts, S);
  __syncthreads();
  stamp<ST>(S, 3);
  const float* hrow = routed ? S.gu + (size_t)wave * L.I
                             : S.gu + (size_t)L.K * L.I + (size_t)(wave - L.K) * half;
  RowStage<kNarrow> Hr;
  load_row<kNarrow, kCoherent>(Hr, hrow, n, lane);
  store_row(Hr, sm.hl[wave], n, lane);  // each wave reads back its own row only
  float r0, r1;
  dot_rows(P, n, sm.hl[wave], nullptr, nullptr, r0, r1);
  stamp<ST>(S, 4);
  if ((lane & 15) == 0) {
    sm.yl[wave][q] = r0;
    sm.yl[wave][q + 4] = r1;
  }
  __syncthreads();
  if (wave == 0 && lane < 8) {
    float acc = sm.yl[L.K][lane] + sm.yl[L.K + 1][lane];
#pragma unroll
    for (int j = 0; j < kMaxK; j++)
      if (j < L.K) acc = acc + sm.pw[j] * sm.yl[j][lane];
    if (residual) acc = res_f + acc;
    out[f0 + lane] = acc;
  }
  stamp<ST>(S, 5);
}

constexpr int kBlockWaves = kUpWaves > kMaxK + 2 ? kUpWaves : kMaxK + 2;

template <int KH, bool ST>
__global__ __launch_bounds__(64 * kBlockWaves) void rows_decode_kernel(DeviceLayer L, Scratch S,
                                                                  const float* residual, float* out) {
  __shared__ __align__(16) DecodeSmem sm;
  // Wave-uniform (scalar) so the per-wave buffer bases stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const DecodeGrid G(L);
  const SyncMap M(S.sync, G);
  int b = blockIdx.x;
  if (b < G.n_logit) {
    if (wave == 0) logit_role<KH, ST>(L, S, sm.up, M, G, b, lane);
    return;
  }
  b -= G.n_logit;
  if (b < G.n_up()) {
    if (wave < kUpWaves) gateup_role<KH, ST>(L, S, sm.up, M, G, b, wave, lane);
    return;
  }
  b -= G.n_up();
  if (wave < L.K + 2) down_role<ST>(L, S, sm.down, M, G, b, residual, out, wave, lane);
}

template <int KH>
void launch_width(const DeviceLayer& L, const Scratch& S, const float* residual, float* out,
                  hipStream_t s) {
  const DecodeGrid G(L);
  const int waves = L.K + 2 > kUpWaves ? L.K + 2 : kUpWaves;
  if (S.stamps)
    rows_decode_kernel<KH, true><<<dim3(G.blocks()), dim3(64 * waves), 0, s>>>(L, S, residual, out);
  else
    rows_decode_kernel<KH, false><<<dim3(G.blocks()), dim3(64 * waves), 0, s>>>(L, S, residual, out);
}

}  // namespace

bool rows_decode_supported(const DeviceLayer& L) {
  // BF16 weights only (INT8 overlays take the split-K engine). Gate/up rows reduce over H (<= 2048), 32 hidden values per workgroup;
  // the down workgroups reduce over I (<= 1024, one wave per routed expert)
  // and the two halves of S (<= 2048, each a whole number of 32-blocks);
  // routing is one wave over E <= 64 logits.
  // The sync words: 1 + 16 counter lines and a flag line per waiting
  // workgroup (K I/32 + 2 H/8 <= 768) fit kDecodeSyncBytes.
  static_assert((1 + kSubCounts + kMaxK * kNarrow / kHidPerWg + 2 * kWide / 8) * kLine * 4 <=
                    (int)kDecodeSyncBytes,
                "decode sync words");
  static_assert(kSubCounts <= kLine, "a down workgroup's sub-set flags share one line");
  static_assert(kLogitsPerWg == 8 && kHidPerWg == 32,
                "the timeline's row count (UOCR_DECODE_STAMP_ROWS) follows these widths");
  return L.quant_mode == 0 && L.H <= kWide && L.S <= kWide && L.I <= kNarrow && L.K >= 1 &&
         L.K <= kMaxK && L.E <= 64 && L.H % 8 == 0 && L.I % kHidPerWg == 0 &&
         L.S % kHidPerWg == 0 && L.S % 64 == 0;
}

void launch_rows_decode(const DeviceLayer& L, const Scratch& S, const float* residual, float* out,
                        hipStream_t s) {
  if (L.H <= 1280)
    launch_width<1280>(L, S, residual, out, s);
  else
    launch_width<kWide>(L, S, residual, out, s);
}

}  // namespace uocr
