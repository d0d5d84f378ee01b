// C-ABI implementation: context, layer upload/repack, forward orchestration.
//
// The layer handle replaces what Decoder::experts reads through projection()
// (src/decoder/mod.rs:99-220): the router, the routed experts and the fused
// shared expert, BF16 or INT8 block-32. The context mirrors CpuContext
// (src/cpu/mod.rs:18-79): a device, a stream and a scratch budget.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/uocr_moe.h"
#include "moe_kernels.hpp"

using uocr::DeviceLayer;
using uocr::Scratch;

// The static scratch of uocr_moe_forward_static (one copy per GPU).
static __device__ __align__(256) char scratch[UOCR_STATIC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  int status = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? UOCR_ERR_RESOURCE
               : (e == hipErrorInvalidDevice || e == hipErrorNoDevice ||
                  e == hipErrorNoBinaryForGpu)
                   ? UOCR_ERR_UNSUPPORTED
                   : UOCR_ERR_RESOURCE;
  return fail(status, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                   \
  do {                                        \
    hipError_t _e = (expr);                   \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

std::once_flag g_attr_once;

}  // namespace

namespace uocr::host {
// Records the message that uocr_last_error returns on this thread.
int set_last_error(int status, const char* message) {
  g_last_error = message;
  return status;
}
}  // namespace uocr::host

enum Phase { kRouter, kTopk, kDispatch, kSplit, kGateUp, kDown, kCombine, kNorm, kDecode, kPhases };
static const char* const kPhaseNames[kPhases] = {"router", "topk",    "dispatch", "split", "gateup",
                                                 "down",   "combine", "norm",     "decode"};

// The context's flag allocation: the device error flag at byte 0, the
// decode engine's cross-workgroup words (zeroed once, zero again after
// every launch) from byte kSyncOffset, then its down partials (all bits
// set once, and again after every launch) from byte kPartOffset.
constexpr size_t kSyncOffset = 256;
constexpr size_t kPartOffset = kSyncOffset + uocr::kDecodeSyncBytes;
constexpr size_t kFlagBytes = kPartOffset + uocr::kDecodePartBytes;

struct uocr_gpu_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  // Second stream of the MFMA engine: the shared expert's GEMMs run there,
  // forked after the input planes and joined before the combine.
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  char* scratch = nullptr;
  size_t scratch_limit = 0;
  int* err = nullptr;       // device error flag
  int* err_host = nullptr;  // pinned readback
  int wait_limit = -1;      // decode engine's wait bound in polls (< 0: its default)
  // Phase timing: bit i of timing_mask enables phase i.
  uint32_t timing_mask = 0;
  std::vector<hipEvent_t> free_events;
  struct Pending {
    int phase;
    hipEvent_t start, stop;
  };
  std::vector<Pending> pending;
  int open_phase = -1;
  hipEvent_t open_start = nullptr;
  uint64_t launches[kPhases] = {};
  double total_ms[kPhases] = {};
};

namespace {

hipEvent_t take_event(uocr_gpu_ctx* ctx) {
  if (!ctx->free_events.empty()) {
    hipEvent_t e = ctx->free_events.back();
    ctx->free_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  (void)hipEventCreate(&e);
  return e;
}

// Brackets the launches between begin and end with events when timing.
void phase_begin(uocr_gpu_ctx* ctx, int phase) {
  if (!ctx || !((ctx->timing_mask >> phase) & 1u)) return;
  ctx->open_phase = phase;
  ctx->open_start = take_event(ctx);
  (void)hipEventRecord(ctx->open_start, ctx->stream);
}

void phase_end(uocr_gpu_ctx* ctx) {
  if (!ctx || ctx->open_phase < 0) return;
  hipEvent_t stop = take_event(ctx);
  (void)hipEventRecord(stop, ctx->stream);
  ctx->pending.push_back({ctx->open_phase, ctx->open_start, stop});
  ctx->open_phase = -1;
}

// Folds completed event pairs into the totals (the stream is synchronised).
void collect_timings(uocr_gpu_ctx* ctx) {
  for (auto& p : ctx->pending) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      ctx->launches[p.phase] += 1;
      ctx->total_ms[p.phase] += ms;
    }
    ctx->free_events.push_back(p.start);
    ctx->free_events.push_back(p.stop);
  }
  ctx->pending.clear();
}

}  // namespace

struct uocr_lm_head {
  int device = 0;
  uocr::LmHeadView view{};
  std::vector<void*> allocations;
  size_t bytes = 0;
};

struct uocr_moe_layer {
  uocr_moe_config cfg{};
  DeviceLayer dev{};
  int device = 0;
  int quant_mode = UOCR_QUANT_NONE;
  std::vector<void*> allocations;
  size_t bytes = 0;
};

namespace {

struct ScratchPlan {
  size_t logits, ids, w, offsets, perm_rows, perm_w, inv_pos, tiles, counters, chunk_counts,
      tile_desc, h, hs, y, ys, xn, xb, gu, q8x, q8s, router_part, total;
};

ScratchPlan plan_scratch(const uocr_moe_config& c, size_t T) {
  const size_t E = c.n_routed_experts, K = c.num_experts_per_tok, H = c.hidden_size;
  const size_t I = c.moe_intermediate_size, S = I * c.n_shared_experts;
  ScratchPlan p{};
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at += align256(bytes ? bytes : 1);
    return here;
  };
  p.logits = take(T * E * 4);
  p.ids = take(T * K * 4);
  p.w = take(T * K * 4);
  p.offsets = take((E + 1) * 4);
  p.perm_rows = take(T * K * 4);
  p.perm_w = take(T * K * 4);
  p.inv_pos = take(T * K * 4);
  // Worst tile count over both engines (one-row tiles for decode).
  p.tiles = take((size_t)uocr::max_tiles((int)T, (int)K, (int)E, 1) * 2 * 4);
  p.counters = take(16);
  p.chunk_counts = take((T + 15) / 16 * 64 * 4);
  p.tile_desc = take(T <= (size_t)uocr::kGemvChunk ? E * uocr::kTileDescInts * 4 : 0);
  p.h = take(T * K * I * 4);
  p.hs = take(T * S * 4);
  p.y = take(T * K * H * 4);
  p.ys = take(T * H * 4);
  p.xn = take(T * H * 4);
  p.xb = take(T * H * 4);
  p.gu = take((T * K * 2 * I + T * 2 * S) * 4);
  // Int8 mode: the quantised input [T, H] and hidden rows [T*K*I + T*S],
  // and their block scales.
  const size_t q8_elems = T * H + T * K * I + T * S;
  p.q8x = take(q8_elems);
  p.q8s = take(q8_elems / 32 * 4);
  // The router's partial logits when it splits H (few tokens).
  p.router_part = take(uocr::router_part_bytes((int)T, (int)H));
  p.total = at;
  return p;
}

// Where a forward runs: a scratch region and its size, the stream, the
// device error flag, and the context whose phase timers apply (null: none).
// side / fork / join: the second stream for the shared expert's GEMMs and
// its events (side null: one stream). Phase timing keeps one stream so
// that every phase's events bracket its own kernels.
struct Exec {
  char* scratch;
  size_t limit;
  hipStream_t stream;
  int* err;
  uocr_gpu_ctx* timing;
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  int* sync = nullptr;  // the decode engine's cross-workgroup words (zero between launches)
  float* part = nullptr;  // the decode engine's down partials (all bits set between launches)
  int wait_limit = -1;  // the decode engine's wait bound in polls (< 0: its default)
};

Exec exec_of(uocr_gpu_ctx* ctx) {
  Exec ex{ctx->scratch, ctx->scratch_limit, ctx->stream, ctx->err, ctx};
  ex.sync = reinterpret_cast<int*>(reinterpret_cast<char*>(ctx->err) + kSyncOffset);
  ex.part = reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->err) + kPartOffset);
  ex.wait_limit = ctx->wait_limit;
  if (ctx->timing_mask == 0) {
    ex.side = ctx->side;
    ex.fork = ctx->fork;
    ex.join = ctx->join;
  }
  return ex;
}

Scratch carve(const Exec& ex, const ScratchPlan& p) {
  Scratch s{};
  char* b = ex.scratch;
  s.logits = reinterpret_cast<float*>(b + p.logits);
  s.topk_ids = reinterpret_cast<int*>(b + p.ids);
  s.topk_w = reinterpret_cast<float*>(b + p.w);
  s.offsets = reinterpret_cast<int*>(b + p.offsets);
  s.perm_rows = reinterpret_cast<int*>(b + p.perm_rows);
  s.perm_w = reinterpret_cast<float*>(b + p.perm_w);
  s.inv_pos = reinterpret_cast<int*>(b + p.inv_pos);
  s.tiles = reinterpret_cast<int*>(b + p.tiles);
  s.counters = reinterpret_cast<int*>(b + p.counters);
  s.chunk_counts = reinterpret_cast<int*>(b + p.chunk_counts);
  s.tile_desc = nullptr;  // set where the small router writes them
  s.h = reinterpret_cast<float*>(b + p.h);
  s.hs = reinterpret_cast<float*>(b + p.hs);
  s.y = reinterpret_cast<float*>(b + p.y);
  s.ys = reinterpret_cast<float*>(b + p.ys);
  s.xn = reinterpret_cast<float*>(b + p.xn);
  s.xb = reinterpret_cast<uint16_t*>(b + p.xb);
  s.gu = reinterpret_cast<float*>(b + p.gu);
  s.q8x = reinterpret_cast<int8_t*>(b + p.q8x);
  s.q8s = reinterpret_cast<float*>(b + p.q8s);
  s.router_part = reinterpret_cast<float*>(b + p.router_part);
  s.err = ex.err;
  s.sync = ex.sync;
  s.part = ex.part;
  s.wait_limit = ex.wait_limit;
  return s;
}

int validate_config(const uocr_moe_config* c) {
  if (!c) return fail(UOCR_ERR_SHAPE, "missing config");
  // ModelConfig::from_json (src/model/config.rs:88-111) for the MoE fields.
  if (c->hidden_size == 0 || c->moe_intermediate_size == 0 || c->n_shared_experts == 0 ||
      c->num_experts_per_tok == 0 || c->num_experts_per_tok > c->n_routed_experts ||
      !std::isfinite(c->rms_norm_eps) || c->rms_norm_eps <= 0.f ||
      !std::isfinite(c->routed_scaling_factor) || c->routed_scaling_factor <= 0.f)
    return fail(UOCR_ERR_SHAPE, "invalid decoder configuration");
  if (c->hidden_size % 64 || c->moe_intermediate_size % 64 || c->n_routed_experts > 64 ||
      c->num_experts_per_tok > 8)
    return fail(UOCR_ERR_UNSUPPORTED,
                "GPU layer needs hidden and intermediate sizes that are multiples of 64, "
                "<= 64 experts and <= 8 experts per token");
  return UOCR_OK;
}

// Most tokens one forward may carry. The MFMA engine addresses its bf16
// activation planes through buffer resources whose ranges and per-lane
// offsets are 32-bit byte counts, with offset 2^31 standing for "outside
// every resource": the x planes (T*H*2 bytes), the routed hidden planes
// (T*K*I*2) and the shared hidden planes (T*S*2) must each stay below
// 2^31 bytes. Expert outputs [T*K, H] are indexed with 32-bit element
// offsets in places, so T*K*H stays below 2^31 too.
size_t max_tokens(const uocr_moe_config& c) {
  const uint64_t H = c.hidden_size, K = c.num_experts_per_tok, I = c.moe_intermediate_size;
  const uint64_t S = I * c.n_shared_experts;
  uint64_t per = 2 * H;
  per = std::max<uint64_t>(per, 2 * K * I);
  per = std::max<uint64_t>(per, 2 * S);
  per = std::max<uint64_t>(per, K * H);
  if (per == 0) return 0;
  return (size_t)(((1ull << 31) - 1) / per);
}

hipMemcpyKind kind_of(uocr_memory where) {
  return where == UOCR_MEMORY_DEVICE ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
}

// Gate/up rows interleaved in blocks of 32: destination rows
// [64b, 64b+32) <- gate [32b, 32b+32), [64b+32, 64b+64) <- up.
int upload_interleaved(char* dst, const void* gate, const void* up, size_t rows, size_t row_bytes,
                       hipMemcpyKind kind, hipStream_t s) {
  const size_t blk = 32 * row_bytes;
  HIP_TRY(hipMemcpy2DAsync(dst, 2 * blk, gate, blk, blk, rows / 32, kind, s), "upload gate");
  HIP_TRY(hipMemcpy2DAsync(dst + blk, 2 * blk, up, blk, blk, rows / 32, kind, s), "upload up");
  return UOCR_OK;
}

__global__ void widen_bf16_kernel(const uint16_t* in, float* out, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = __uint_as_float((uint32_t)in[i] << 16);
}

// Int8Matrix::from_parts / QuantizedWeights::load value rules
// (src/cpu/quantized.rs:31-35, 351): byte 0x80 (-128) is rejected as
// Format, non-finite or negative scales as Numerical.
__global__ void check_int8_kernel(const int8_t* q, size_t nq, const float* s, size_t ns,
                                  int* flag) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nq; i += stride)
    if (q[i] == -128) atomicMax(flag, UOCR_ERR_FORMAT);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < ns; i += stride)
    if (!isfinite(s[i]) || s[i] < 0.f) atomicMax(flag, UOCR_ERR_NUMERICAL);
}

int read_and_clear_error(uocr_gpu_ctx* ctx) {
  HIP_TRY(hipMemcpyAsync(ctx->err_host, ctx->err, sizeof(int), hipMemcpyDeviceToHost,
                         ctx->stream),
          "read device error flag");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "synchronize");
  int e = *ctx->err_host;
  if (e != 0) {
    // The decode engine's words and partials too: a wait that gave up
    // (Resource) can leave a flag or a partial that its producer set later.
    HIP_TRY(hipMemsetAsync(ctx->err, 0, kPartOffset, ctx->stream), "clear device error flag");
    HIP_TRY(hipMemsetAsync(reinterpret_cast<char*>(ctx->err) + kPartOffset, 0xff,
                           uocr::kDecodePartBytes, ctx->stream),
            "reset the decode partials");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "synchronize");
    return fail(e, e == UOCR_ERR_NUMERICAL  ? "nonfinite numerical input on device"
                   : e == UOCR_ERR_RESOURCE ? "a one-token launch's cross-workgroup wait reached its bound"
                                            : "device reported an error");
  }
  return UOCR_OK;
}

// Engine of a forward: the one-token decode engine, the small-batch engine
// (row tiles of <= 16 tokens, bandwidth-bound) for T <= 16, the MFMA
// grouped GEMM for larger batches (INT8 overlays streamed as int8 rows and
// dequantised in registers; under DynamicActivations the single-row groups
// still take the small-batch engine's W8A8 path).
enum class Engine { Decode, Batch, Mfma, Int8 };

Engine choose_engine(const uocr_moe_layer* layer, size_t T, uint32_t flags) {
  const DeviceLayer& L = layer->dev;
  // The opt-in int8 mode: every group W8A8; one token already is on the
  // decode engine.
  if (flags & UOCR_FLAG_INT8_MFMA)
    return T == 1 && uocr::decode_supported(L) ? Engine::Decode : Engine::Int8;
  const bool mfma = (flags & UOCR_FLAG_FORCE_MFMA) ||
                    (!(flags & UOCR_FLAG_FORCE_GEMV) && T > (size_t)uocr::kGemvChunk);
  if (mfma) return Engine::Mfma;
  if (T == 1 && uocr::decode_supported(L)) return Engine::Decode;
  // Shapes beyond the small-batch engine's registers take the grouped GEMM
  // unless the caller forces the small-batch engine.
  if (!uocr::batch_supported(L) && !(flags & UOCR_FLAG_FORCE_GEMV)) return Engine::Mfma;
  return Engine::Batch;
}

// bf16 planes of the layer input in scratch (the MFMA engine's A operand).
void input_planes(const Scratch& S, const DeviceLayer& L, size_t T, uint32_t flags, uint16_t** hi,
                  uint16_t** lo) {
  *hi = S.xb;
  *lo = (flags & UOCR_FLAG_BF16_ACTIVATIONS) ? nullptr : S.xb + T * L.H;
}

// planes_ready: the MFMA engine's input planes are already in scratch.
// next: the following layer's RMSNorm, fused into this layer's combine (not
// taken by the decode engine; *fused says whether it ran).
int enqueue_experts(const Exec& ex, const uocr_moe_layer* layer, const float* x, size_t T,
                    const float* residual, float* y, uint32_t flags,
                    const uocr_moe_trace* trace, bool x_in_scratch, bool planes_ready = false,
                    const uocr::RowNorm* next = nullptr, bool* fused = nullptr) {
  if (fused) *fused = false;
  uocr_gpu_ctx* ctx = ex.timing;  // phase timers only
  const uocr_moe_config& c = layer->cfg;
  const ScratchPlan plan = plan_scratch(c, T);
  if (plan.total > ex.limit)
    return fail(UOCR_ERR_RESOURCE, "operation exceeds scratch limit (%zu > %zu bytes)",
                plan.total, ex.limit);
  Scratch S = carve(ex, plan);
  if (!x_in_scratch) S.xn = const_cast<float*>(x);
  const DeviceLayer& L = layer->dev;
  const int Ti = (int)T;
  hipStream_t st = ex.stream;
  const uocr_w8a8_trace* q8t =
      trace && L.quant_mode == UOCR_QUANT_DYNAMIC_ACTIVATIONS ? trace->w8a8 : nullptr;
  static_assert(uocr::kDecodeStamps == UOCR_DECODE_STAMPS, "decode timeline row");
  if (trace) S.stamps = reinterpret_cast<unsigned long long*>(trace->decode_stamps);
  if (q8t) {
    S.q8.gateup = q8t->gateup_sums;
    S.q8.down = q8t->down_sums;
    S.q8.hidden = q8t->hidden;
    if (T == 1) {
      S.q8.s_gateup = q8t->shared_gateup_sums;
      S.q8.s_down = q8t->shared_down_sums;
      S.q8.s_hidden = q8t->shared_hidden;
    }
  }
  // The W8A8 trace's hidden rows, copied where the engine holds them (the
  // MFMA GEMMs later reuse the small-batch engine's hidden rows' bytes).
  auto trace_hidden = [&](const float* routed, const float* shared) -> int {
    if (S.q8.hidden)
      HIP_TRY(hipMemcpyAsync(S.q8.hidden, routed, T * L.K * L.I * 4, hipMemcpyDeviceToDevice, st),
              "trace copy");
    if (S.q8.s_hidden)
      HIP_TRY(hipMemcpyAsync(S.q8.s_hidden, shared, (size_t)L.S * 4, hipMemcpyDeviceToDevice, st),
              "trace copy");
    return UOCR_OK;
  };
  if ((flags & UOCR_FLAG_INT8_MFMA) && L.quant_mode != UOCR_QUANT_DYNAMIC_ACTIVATIONS)
    return fail(UOCR_ERR_UNSUPPORTED,
                "int8 activations need an INT8 overlay in DynamicActivations mode");
  const Engine engine = choose_engine(layer, T, flags);
  if (engine == Engine::Int8 && !uocr::i8_supported(L))
    return fail(UOCR_ERR_UNSUPPORTED, "int8 engine needs widths that are multiples of 64");
  const bool mfma = engine == Engine::Mfma;
  const bool int8 = engine == Engine::Int8;
  // The small-batch engine also takes the single-row W8A8 groups of the
  // MFMA engine.
  if ((!mfma || L.quant_mode == UOCR_QUANT_DYNAMIC_ACTIVATIONS) && !uocr::batch_supported(L))
    return fail(UOCR_ERR_UNSUPPORTED,
                "small-batch engine needs widths <= 2048, expert and shared widths that are "
                "multiples of 16 and a hidden width that is a multiple of 32");
  const bool bf16_only = (flags & UOCR_FLAG_BF16_ACTIVATIONS) != 0;
  // Row tiles: 256 rows on the MFMA engine with BF16 weights (an expert's
  // last tile of <= 128 rows runs as 128 x 512 items), 64 rows with INT8
  // weights (64 x 512 items) and in the int8 mode, 16 on the small-batch
  // engine.
  const bool q8 = L.quant_mode != UOCR_QUANT_NONE;
  const int bm = mfma ? (q8 ? uocr::kMfmaQ8BM : uocr::kMfmaBM)
                      : int8 ? uocr::kI8BM : uocr::kGemvChunk;
  const int narrow = mfma && !q8 ? uocr::kMfmaBM / 2 : 0;
  const int tiles_bound = uocr::max_tiles(Ti, L.K, L.E, bm);
  if (tiles_bound > 65535)
    return fail(UOCR_ERR_RESOURCE, "token count too large for one forward (%zu)", T);
  if (engine == Engine::Decode) {
    // One token: one launch, its workgroups ordered by the words at S.sync.
    if (!S.sync || !S.part)
      return fail(UOCR_ERR_UNSUPPORTED, "decode engine without its sync words");
    phase_begin(ctx, kDecode);
    uocr::launch_decode(L, S, residual, y, st);
    phase_end(ctx);
    if (int r = trace_hidden(S.gu, S.gu + (size_t)L.K * L.I)) return r;
  } else {
    // MFMA engine: the input planes, then (two streams) the shared expert's
    // gate/up and down on the side stream, which needs no routing, while
    // this stream routes and runs the routed experts; each launch's last
    // round of items then overlaps the other stream's work. It pays where
    // those tails are a large share (1024-token Zipf layer 0.257 -> 0.235
    // ms) and costs at 4096 tokens (12-layer stack 6.25 -> 6.52 ms: with two
    // kernels resident, a launch's workgroups no longer reach the XCDs in
    // the order its item split assumes), so it is limited to
    // kOverlapMaxTokens tokens.
    constexpr size_t kOverlapMaxTokens = 2048;
    uocr::MfmaPlanes P{};
    // (Under DynamicActivations the small-batch engine's single-row pass on
    // this stream touches only routed rows' hidden and output buffers.)
    // Under DynamicActivations one token makes the shared expert a
    // single-row group as well (src/decoder/mod.rs:103-104): with the MFMA
    // engine forced at T = 1 it runs as W8A8 on the small-batch engine's
    // shared units, and the MFMA launches take the routed items only.
    const bool shared_single = mfma && T == 1 && L.quant_mode == UOCR_QUANT_DYNAMIC_ACTIVATIONS;
    const bool overlap = mfma && ex.side && L.S > 0 && T <= kOverlapMaxTokens && !shared_single;
    if (mfma) {
      P.x_hi = S.xb;
      P.x_lo = S.xb + T * L.H;
      P.h_hi = reinterpret_cast<uint16_t*>(S.h);
      P.h_lo = P.h_hi + T * L.K * L.I;
      P.hs_hi = reinterpret_cast<uint16_t*>(S.hs);
      P.hs_lo = P.hs_hi + T * L.S;
    }
    // One stream: the fused MFMA router writes the planes itself (it reads
    // every value of x once anyway), so no split launch precedes it. Two
    // streams keep the split first, so that the fork comes before the
    // routing and the shared expert's GEMMs reach the CUs ahead of the
    // routed ones (forking after the router took the 512-token INT8 layer
    // from 0.165 to 0.199 ms; forking first with a side-stream copy of the
    // planes measured the same as the split here).
    const bool fused_router = T > (size_t)uocr::kGemvChunk && uocr::router_mfma_supported(L.H);
    const bool router_planes = mfma && !planes_ready && fused_router && !overlap;
    if (mfma && !planes_ready && !router_planes) {
      phase_begin(ctx, kSplit);
      uocr::launch_split_planes(S.xn, Ti, L.H, P.x_hi, bf16_only ? nullptr : P.x_lo, st);
      phase_end(ctx);
    }
    if (overlap) {
      const int shared_tiles = (Ti + bm - 1) / bm;
      HIP_TRY(hipEventRecord(ex.fork, st), "fork event");
      HIP_TRY(hipStreamWaitEvent(ex.side, ex.fork, 0), "fork wait");
      uocr::launch_mfma_gateup(L, S, P, Ti, shared_tiles, bf16_only, uocr::kListShared, ex.side);
      uocr::launch_mfma_down(L, S, P, Ti, shared_tiles, bf16_only, uocr::kListShared, ex.side);
      HIP_TRY(hipEventRecord(ex.join, ex.side), "join event");
    }
    if (T <= (size_t)uocr::kGemvChunk && !mfma && !int8) {
      // Few tokens: one launch; the last of its logit workgroups routes
      // every token and builds the dispatch (counted in a word at S.sync).
      if (!S.sync) return fail(UOCR_ERR_UNSUPPORTED, "small-batch router without its sync word");
      S.tile_desc = reinterpret_cast<int*>(ex.scratch + plan.tile_desc);
      phase_begin(ctx, kRouter);
      uocr::launch_small_route(S.xn, L, S, Ti, st);
      phase_end(ctx);
    } else if (fused_router) {
      // Many tokens: fused MFMA router + top-k, then the chunked dispatch.
      phase_begin(ctx, kRouter);
      uocr::launch_router_topk_mfma(S.xn, L.router, Ti, L.H, L.E, L.K, L.normalize, L.scale,
                                    S.logits, S.topk_ids, S.topk_w, S.chunk_counts,
                                    router_planes ? P.x_hi : nullptr,
                                    router_planes && !bf16_only ? P.x_lo : nullptr, S.err,
                                    S.router_part, S.sync ? S.sync + uocr::kRouterSyncWord : nullptr,
                                    st);
      phase_end(ctx);
      phase_begin(ctx, kDispatch);
      uocr::launch_dispatch_chunked(S.topk_ids, S.topk_w, Ti, L.E, L.K, bm, narrow, S.chunk_counts,
                                    S.offsets, S.perm_rows, S.perm_w, S.inv_pos, S.tiles,
                                    S.counters, st);
      phase_end(ctx);
    } else {
      // MFMA engine forced on a small batch, or a hidden width beyond the
      // fused router's.
      phase_begin(ctx, kRouter);
      uocr::launch_router_logits(S.xn, L.router, Ti, L.H, L.E, S.logits, st);
      phase_end(ctx);
      phase_begin(ctx, kTopk);
      uocr::launch_topk(S.logits, Ti, L.E, L.K, L.normalize, L.scale, S.topk_ids, S.topk_w,
                        S.err, st);
      phase_end(ctx);
      phase_begin(ctx, kDispatch);
      uocr::launch_dispatch(S.topk_ids, S.topk_w, Ti, L.E, L.K, bm, narrow, S.offsets, S.perm_rows,
                            S.perm_w, S.inv_pos, S.tiles, S.counters, st);
      phase_end(ctx);
    }
    if (int8) {
      // Quantise the input rows, gate/up into quantised hidden rows (FP32
      // ones and a quantising launch when traced), down.
      uocr::I8Planes P;
      const size_t routed_rows = T * L.K;
      P.xq = S.q8x;
      P.xs = S.q8s;
      P.hid = S.h;
      P.hid_shared = S.hs;
      P.hid_q = S.q8x + T * L.H;
      P.hid_s = S.q8s + T * L.H / 32;
      phase_begin(ctx, kSplit);
      uocr::launch_quantize_rows(S.xn, Ti, L.H, S.q8x, S.q8s, nullptr, 0, 32, nullptr, nullptr,
                                 S.err, st);
      phase_end(ctx);
      phase_begin(ctx, kGateUp);
      uocr::launch_i8_gateup(L, S, P, Ti, tiles_bound, st);
      phase_end(ctx);
      // Untraced, the gate/up epilogue has written the hidden rows quantised.
      if (uocr::i8_traced(S, Ti)) {
        if (int r = trace_hidden(S.h, S.hs)) return r;
        phase_begin(ctx, kSplit);
        uocr::launch_quantize_rows(S.h, (int)routed_rows, L.I, P.hid_q, P.hid_s, S.hs, Ti, L.S,
                                   P.hid_q + routed_rows * L.I, P.hid_s + routed_rows * L.I / 32,
                                   S.err, st);
        phase_end(ctx);
      }
      phase_begin(ctx, kDown);
      uocr::launch_i8_down(L, S, P, Ti, tiles_bound, st);
      phase_end(ctx);
    } else if (mfma) {
      if (L.quant_mode == UOCR_QUANT_DYNAMIC_ACTIVATIONS) {
        // W8A8 for groups of one row (src/decoder/mod.rs:103-104): the
        // small-batch engine's single-row pass on this stream (hidden rows
        // in S.gu; the W8A8 trace's hidden rows written by the pass itself).
        // On the second stream, after the shared expert's GEMMs, it
        // lengthened the stream that ends the layer (512-token W8A8 layer
        // 0.162 -> 0.171 ms).
        phase_begin(ctx, kGateUp);
        uocr::launch_singles_gateup(L, S, Ti, st);
        if (shared_single) uocr::launch_batch_gateup(L, S, Ti, tiles_bound, bm, st, true);
        phase_end(ctx);
        phase_begin(ctx, kDown);
        uocr::launch_singles_down(L, S, Ti, st);
        if (shared_single) uocr::launch_batch_down(L, S, Ti, tiles_bound, bm, st, true);
        phase_end(ctx);
      }
      const int lists = overlap || shared_single ? uocr::kListRouted : uocr::kListAll;
      phase_begin(ctx, kGateUp);
      uocr::launch_mfma_gateup(L, S, P, Ti, tiles_bound, bf16_only, lists, st);
      phase_end(ctx);
      phase_begin(ctx, kDown);
      uocr::launch_mfma_down(L, S, P, Ti, tiles_bound, bf16_only, lists, st);
      phase_end(ctx);
      if (overlap) HIP_TRY(hipStreamWaitEvent(st, ex.join, 0), "join wait");
    } else {
      // (The W8A8 trace's hidden rows of single-row groups are written by
      // the gate/up units themselves.)
      phase_begin(ctx, kGateUp);
      uocr::launch_batch_gateup(L, S, Ti, tiles_bound, bm, st);
      phase_end(ctx);
      phase_begin(ctx, kDown);
      uocr::launch_batch_down(L, S, Ti, tiles_bound, bm, st);
      phase_end(ctx);
    }
    phase_begin(ctx, kCombine);
    uocr::launch_combine(S, residual, Ti, L.H, L.K, y, next,
                         mfma && bf16_only && L.quant_mode == UOCR_QUANT_NONE, st);
    phase_end(ctx);
    if (fused) *fused = next != nullptr;
  }
  HIP_TRY(hipGetLastError(), "kernel launch");
  if (trace) {
    const size_t TK = T * L.K;
    auto copy = [&](void* dst, const void* src, size_t bytes) -> int {
      if (dst) HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st), "trace copy");
      return UOCR_OK;
    };
    int r;
    if ((r = copy(trace->logits, S.logits, T * L.E * 4))) return r;
    if ((r = copy(trace->topk_ids, S.topk_ids, TK * 4))) return r;
    if ((r = copy(trace->topk_weights, S.topk_w, TK * 4))) return r;
    if ((r = copy(trace->expert_offsets, S.offsets, (L.E + 1) * 4))) return r;
    if ((r = copy(trace->perm_rows, S.perm_rows, TK * 4))) return r;
    if ((r = copy(trace->perm_weights, S.perm_w, TK * 4))) return r;
  }
  return UOCR_OK;
}

// ------------------------------------------------ allocation-free forward
//
// Scratch of uocr_moe_forward_static: one array of UOCR_STATIC_SCRATCH_BYTES
// per GPU, held until the process ends. Its first kStaticFlagBytes hold the
// device error flag when the caller passes none and, from byte kSyncOffset,
// the decode engine's cross-workgroup words (cleared at every call); the
// forward's scratch follows. In
// host code `scratch` only names the host-side stand-in: the device address
// comes from hipGetSymbolAddress, once per device, and only that address is
// ever passed to kernels.

constexpr int kMaxStaticDevices = 64;
constexpr size_t kStaticFlagBytes = kFlagBytes;
static_assert(kStaticFlagBytes == UOCR_STATIC_RESERVED_BYTES, "static reservation");
std::mutex g_static_mu;
char* g_static_base[kMaxStaticDevices] = {};

// Clears the error flag and the decode engine's words, and sets every bit
// of its partials, at the start of each static forward (16 bytes per
// thread and pass over the grid).
__global__ void clear_flag_kernel(int* flag, int* sync, float* part) {
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  if (tid == 0) *flag = 0;
  uint4* w = reinterpret_cast<uint4*>(sync);
  for (size_t i = tid; i < uocr::kDecodeSyncBytes / 16; i += stride) w[i] = make_uint4(0, 0, 0, 0);
  uint4* p = reinterpret_cast<uint4*>(part);
  const uint4 ones = make_uint4(~0u, ~0u, ~0u, ~0u);
  for (size_t i = tid; i < uocr::kDecodePartBytes / 16; i += stride) p[i] = ones;
}

// The device address of this device's array (the device must be current).
int static_scratch_of(int device, char** out) {
  std::lock_guard<std::mutex> lock(g_static_mu);
  if (device < 0 || device >= kMaxStaticDevices)
    return fail(UOCR_ERR_UNSUPPORTED, "static scratch supports devices 0..%d", kMaxStaticDevices - 1);
  if (!g_static_base[device]) {
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "static scratch address");
    g_static_base[device] = static_cast<char*>(p);
  }
  *out = g_static_base[device];
  return UOCR_OK;
}

}  // namespace

extern "C" {

int uocr_gpu_ctx_create(int device, size_t scratch_limit, uocr_gpu_ctx** out) {
  if (!out) return fail(UOCR_ERR_SHAPE, "null output handle");
  *out = nullptr;
  if (scratch_limit == 0) return fail(UOCR_ERR_RESOURCE, "scratch limit must be nonzero");
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n), "device count");
  if (device < 0 || device >= n) return fail(UOCR_ERR_UNSUPPORTED, "no GPU device %d", device);
  HIP_TRY(hipSetDevice(device), "set device");
  std::call_once(g_attr_once, [] {
    uocr::gemv_init_attributes();
    uocr::mfma_init_attributes();
  });
  auto* ctx = new uocr_gpu_ctx();
  ctx->device = device;
  ctx->scratch_limit = scratch_limit;
  hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking);
  // fork/join only order the two streams of this device, so a device-scope release is
  // enough: no system-scope cache write-back and invalidate at each record.
  const unsigned ev_flags = hipEventDisableTiming | hipEventDisableSystemFence;
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->fork, ev_flags);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->join, ev_flags);
  if (e == hipSuccess) e = hipMalloc(&ctx->scratch, scratch_limit);
  if (e == hipSuccess) e = hipMalloc(&ctx->err, kFlagBytes);
  if (e == hipSuccess) e = hipHostMalloc(&ctx->err_host, sizeof(int));
  if (e == hipSuccess) e = hipMemset(ctx->err, 0, kPartOffset);
  if (e == hipSuccess)
    e = hipMemset(reinterpret_cast<char*>(ctx->err) + kPartOffset, 0xff, uocr::kDecodePartBytes);
  if (e != hipSuccess) {
    uocr_gpu_ctx_destroy(ctx);
    return hip_fail(e, "context allocation");
  }
  *out = ctx;
  return UOCR_OK;
}

void uocr_gpu_ctx_destroy(uocr_gpu_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->side) (void)hipStreamSynchronize(ctx->side);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->err) (void)hipFree(ctx->err);
  if (ctx->err_host) (void)hipHostFree(ctx->err_host);
  collect_timings(ctx);
  for (hipEvent_t e : ctx->free_events) (void)hipEventDestroy(e);
  if (ctx->fork) (void)hipEventDestroy(ctx->fork);
  if (ctx->join) (void)hipEventDestroy(ctx->join);
  if (ctx->side) (void)hipStreamDestroy(ctx->side);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

void* uocr_gpu_ctx_stream(uocr_gpu_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int uocr_gpu_ctx_synchronize(uocr_gpu_ctx* ctx) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  return read_and_clear_error(ctx);
}

int uocr_gpu_ctx_set_timing(uocr_gpu_ctx* ctx, uint32_t phase_mask) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  ctx->timing_mask = phase_mask;
  return UOCR_OK;
}

int uocr_gpu_ctx_set_wait_limit(uocr_gpu_ctx* ctx, int polls) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  ctx->wait_limit = polls;
  return UOCR_OK;
}

int uocr_gpu_ctx_timings(uocr_gpu_ctx* ctx, uocr_phase_time* out, size_t cap, size_t* count) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "synchronize");
  collect_timings(ctx);
  for (size_t i = 0; i < (size_t)kPhases && i < cap && out; i++) {
    out[i].name = kPhaseNames[i];
    out[i].launches = ctx->launches[i];
    out[i].total_ms = ctx->total_ms[i];
  }
  if (count) *count = kPhases;
  for (int i = 0; i < kPhases; i++) {
    ctx->launches[i] = 0;
    ctx->total_ms[i] = 0.0;
  }
  return UOCR_OK;
}

const char* uocr_last_error(const uocr_gpu_ctx* ctx) {
  (void)ctx;
  return g_last_error.c_str();
}

size_t uocr_moe_scratch_bytes(const uocr_moe_config* cfg, size_t T) {
  if (!cfg) return 0;
  return plan_scratch(*cfg, T).total;
}

size_t uocr_moe_max_tokens(const uocr_moe_config* cfg) {
  if (!cfg) return 0;
  return max_tokens(*cfg);
}

int uocr_moe_layer_create(uocr_gpu_ctx* ctx, const uocr_moe_config* cfg,
                          const uocr_moe_bf16_weights* w, uocr_memory where,
                          uocr_moe_layer** out) {
  if (!out) return fail(UOCR_ERR_SHAPE, "null output handle");
  *out = nullptr;
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  int r = validate_config(cfg);
  if (r) return r;
  if (!w || !w->router || !w->expert_gate || !w->expert_up || !w->expert_down ||
      !w->shared_gate || !w->shared_up || !w->shared_down)
    return fail(UOCR_ERR_FORMAT, "missing MoE weight tensor");
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  auto* layer = new uocr_moe_layer();
  layer->cfg = *cfg;
  layer->device = ctx->device;
  DeviceLayer& L = layer->dev;
  L.H = (int)cfg->hidden_size;
  L.I = (int)cfg->moe_intermediate_size;
  L.S = L.I * (int)cfg->n_shared_experts;
  L.E = (int)cfg->n_routed_experts;
  L.K = (int)cfg->num_experts_per_tok;
  L.normalize = cfg->norm_topk_prob ? 1 : 0;
  L.scale = cfg->routed_scaling_factor;
  L.eps = cfg->rms_norm_eps;
  L.quant_mode = UOCR_QUANT_NONE;
  const size_t H = L.H, I = L.I, S = L.S, E = L.E;
  const size_t n13 = (E * 2 * I + 2 * S) * H, n2 = (E * I + S) * H;
  auto alloc = [&](size_t bytes, void** p) -> hipError_t {
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) {
      layer->allocations.push_back(*p);
      layer->bytes += bytes;
    }
    return e;
  };
  void *router = nullptr, *w13 = nullptr, *w2 = nullptr, *w13k = nullptr, *w2k = nullptr,
       *norm = nullptr;
  hipError_t e = alloc(E * H * 2, &router);
  if (e == hipSuccess) e = alloc(n13 * 2, &w13);
  if (e == hipSuccess) e = alloc(n2 * 2, &w2);
  if (e == hipSuccess) e = alloc(n13 * 2, &w13k);
  if (e == hipSuccess) e = alloc(n2 * 2, &w2k);
  if (e == hipSuccess) e = alloc(H * 4, &norm);
  if (e != hipSuccess) {
    uocr_moe_layer_destroy(layer);
    return hip_fail(e, "layer allocation");
  }
  const hipMemcpyKind kind = kind_of(where);
  hipStream_t st = ctx->stream;
  auto finish = [&](int status) {
    if (status) uocr_moe_layer_destroy(layer);
    return status;
  };
  if ((e = hipMemcpyAsync(router, w->router, E * H * 2, kind, st)) != hipSuccess)
    return finish(hip_fail(e, "upload router"));
  char* d13 = static_cast<char*>(w13);
  for (size_t g = 0; g < E; g++) {
    r = upload_interleaved(d13 + g * 2 * I * H * 2, w->expert_gate + g * I * H,
                           w->expert_up + g * I * H, I, H * 2, kind, st);
    if (r) return finish(r);
  }
  r = upload_interleaved(d13 + E * 2 * I * H * 2, w->shared_gate, w->shared_up, S, H * 2, kind,
                         st);
  if (r) return finish(r);
  if ((e = hipMemcpyAsync(w2, w->expert_down, E * H * I * 2, kind, st)) != hipSuccess)
    return finish(hip_fail(e, "upload down"));
  if ((e = hipMemcpyAsync(static_cast<char*>(w2) + E * H * I * 2, w->shared_down, H * S * 2, kind,
                          st)) != hipSuccess)
    return finish(hip_fail(e, "upload shared down"));
  // The MFMA engine's k-blocked panels of the same matrices.
  uocr::launch_panelize(w13, w13k, 2, (int)(2 * I), (int)H, (int)E, st);
  uocr::launch_panelize(static_cast<char*>(w13) + E * 2 * I * H * 2,
                        static_cast<char*>(w13k) + E * 2 * I * H * 2, 2, (int)(2 * S), (int)H, 1, st);
  uocr::launch_panelize(w2, w2k, 2, (int)H, (int)I, (int)E, st);
  uocr::launch_panelize(static_cast<char*>(w2) + E * H * I * 2, static_cast<char*>(w2k) + E * H * I * 2,
                        2, (int)H, (int)S, 1, st);
  if ((e = hipGetLastError()) != hipSuccess) return finish(hip_fail(e, "weight panels"));
  if (w->norm_weight) {
    void* tmp = nullptr;
    if ((e = hipMalloc(&tmp, H * 2)) != hipSuccess) return finish(hip_fail(e, "norm staging"));
    e = hipMemcpyAsync(tmp, w->norm_weight, H * 2, kind, st);
    if (e == hipSuccess) {
      hipLaunchKernelGGL(widen_bf16_kernel, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, st,
                         (const uint16_t*)tmp, (float*)norm, (int)H);
      e = hipStreamSynchronize(st);
    }
    (void)hipFree(tmp);
    if (e != hipSuccess) return finish(hip_fail(e, "upload norm"));
    L.norm_w = static_cast<const float*>(norm);
  } else {
    L.norm_w = nullptr;
  }
  if ((e = hipStreamSynchronize(st)) != hipSuccess) return finish(hip_fail(e, "upload"));
  L.router = static_cast<const uint16_t*>(router);
  L.w13 = static_cast<const uint16_t*>(w13);
  L.w2 = static_cast<const uint16_t*>(w2);
  L.w13k = static_cast<const uint16_t*>(w13k);
  L.w2k = static_cast<const uint16_t*>(w2k);
  *out = layer;
  return UOCR_OK;
}

int uocr_moe_layer_attach_int8(uocr_gpu_ctx* ctx, uocr_moe_layer* layer,
                               const uocr_moe_int8_weights* w, uocr_memory where,
                               uocr_quant_mode mode) {
  if (!ctx || !layer) return fail(UOCR_ERR_SHAPE, "null handle");
  if (mode != UOCR_QUANT_WEIGHTS_ONLY && mode != UOCR_QUANT_DYNAMIC_ACTIVATIONS) {
    if (mode == UOCR_QUANT_NONE && !w) {
      layer->quant_mode = UOCR_QUANT_NONE;
      layer->dev.quant_mode = UOCR_QUANT_NONE;
      return UOCR_OK;
    }
    return fail(UOCR_ERR_UNSUPPORTED, "unknown quantization mode");
  }
  if (!w || !w->expert_gate || !w->expert_up || !w->expert_down || !w->shared_gate ||
      !w->shared_up || !w->shared_down || !w->expert_gate_scales || !w->expert_up_scales ||
      !w->expert_down_scales || !w->shared_gate_scales || !w->shared_up_scales ||
      !w->shared_down_scales)
    return fail(UOCR_ERR_FORMAT, "dynamic INT8 requires a quantized weight overlay");
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  DeviceLayer& L = layer->dev;
  const size_t H = L.H, I = L.I, S = L.S, E = L.E;
  const size_t n13 = (E * 2 * I + 2 * S) * H, n2 = (E * I + S) * H;
  void *q13 = nullptr, *s13 = nullptr, *q2 = nullptr, *s2 = nullptr, *q13k = nullptr, *q2k = nullptr,
       *s2k = nullptr, *s13k = nullptr;
  std::vector<void*> fresh;
  auto alloc = [&](size_t bytes, void** p) -> hipError_t {
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) fresh.push_back(*p);
    return e;
  };
  auto release = [&](int status) {
    for (void* p : fresh) (void)hipFree(p);
    return status;
  };
  hipError_t e = alloc(n13, &q13);
  if (e == hipSuccess) e = alloc(n13 / 32 * 4, &s13);
  if (e == hipSuccess) e = alloc(n2, &q2);
  if (e == hipSuccess) e = alloc(n2 / 32 * 4, &s2);
  if (e == hipSuccess) e = alloc(n13, &q13k);
  if (e == hipSuccess) e = alloc(n2, &q2k);
  if (e == hipSuccess) e = alloc(n2 / 32 * 4, &s2k);
  if (e == hipSuccess) e = alloc(n13 / 32 * 4, &s13k);
  if (e != hipSuccess) return release(hip_fail(e, "INT8 allocation"));
  const hipMemcpyKind kind = kind_of(where);
  hipStream_t st = ctx->stream;
  char* dq = static_cast<char*>(q13);
  char* ds = static_cast<char*>(s13);
  int r;
  for (size_t g = 0; g < E; g++) {
    if ((r = upload_interleaved(dq + g * 2 * I * H, w->expert_gate + g * I * H,
                                w->expert_up + g * I * H, I, H, kind, st)))
      return release(r);
    if ((r = upload_interleaved(ds + g * 2 * I * (H / 32) * 4,
                                w->expert_gate_scales + g * I * (H / 32),
                                w->expert_up_scales + g * I * (H / 32), I, (H / 32) * 4, kind,
                                st)))
      return release(r);
  }
  if ((r = upload_interleaved(dq + E * 2 * I * H, w->shared_gate, w->shared_up, S, H, kind, st)))
    return release(r);
  if ((r = upload_interleaved(ds + E * 2 * I * (H / 32) * 4, w->shared_gate_scales,
                              w->shared_up_scales, S, (H / 32) * 4, kind, st)))
    return release(r);
  if ((e = hipMemcpyAsync(q2, w->expert_down, E * H * I, kind, st)) != hipSuccess ||
      (e = hipMemcpyAsync(static_cast<char*>(q2) + E * H * I, w->shared_down, H * S, kind, st)) !=
          hipSuccess ||
      (e = hipMemcpyAsync(s2, w->expert_down_scales, E * H * (I / 32) * 4, kind, st)) !=
          hipSuccess ||
      (e = hipMemcpyAsync(static_cast<char*>(s2) + E * H * (I / 32) * 4, w->shared_down_scales,
                          H * (S / 32) * 4, kind, st)) != hipSuccess)
    return release(hip_fail(e, "upload INT8 down"));
  // The MFMA engine's k-blocked panels of the int8 values.
  uocr::launch_panelize(q13, q13k, 1, (int)(2 * I), (int)H, (int)E, st);
  uocr::launch_panelize(static_cast<char*>(q13) + E * 2 * I * H, static_cast<char*>(q13k) + E * 2 * I * H,
                        1, (int)(2 * S), (int)H, 1, st);
  uocr::launch_panelize(q2, q2k, 1, (int)H, (int)I, (int)E, st);
  uocr::launch_panelize(static_cast<char*>(q2) + E * H * I, static_cast<char*>(q2k) + E * H * I, 1,
                        (int)H, (int)S, 1, st);
  // The one-token engine's block-major down scales.
  uocr::launch_transpose_f32(static_cast<const float*>(s2), static_cast<float*>(s2k), (int)H,
                             (int)(I / 32), (int)E, st);
  uocr::launch_transpose_f32(static_cast<const float*>(s2) + E * H * (I / 32),
                             static_cast<float*>(s2k) + E * H * (I / 32), (int)H, (int)(S / 32), 1,
                             st);
  // The MFMA engines' block-major gate/up scales ([H/32][2W] per group).
  uocr::launch_transpose_f32(static_cast<const float*>(s13), static_cast<float*>(s13k),
                             (int)(2 * I), (int)(H / 32), (int)E, st);
  uocr::launch_transpose_f32(static_cast<const float*>(s13) + E * 2 * I * (H / 32),
                             static_cast<float*>(s13k) + E * 2 * I * (H / 32), (int)(2 * S),
                             (int)(H / 32), 1, st);
  // Validate the uploaded values on the device.
  HIP_TRY(hipMemsetAsync(ctx->err, 0, sizeof(int), st), "clear flag");
  hipLaunchKernelGGL(check_int8_kernel, dim3(1024), dim3(256), 0, st, (const int8_t*)q13, n13,
                     (const float*)s13, n13 / 32, ctx->err);
  hipLaunchKernelGGL(check_int8_kernel, dim3(1024), dim3(256), 0, st, (const int8_t*)q2, n2,
                     (const float*)s2, n2 / 32, ctx->err);
  r = read_and_clear_error(ctx);
  if (r) {
    return release(fail(r, r == UOCR_ERR_FORMAT ? "invalid INT8 matrix (byte 128)"
                                                 : "INT8 scales must be finite and nonnegative"));
  }
  // Replace any previous overlay.
  for (void* p : {(void*)L.q13, (void*)L.s13, (void*)L.q2, (void*)L.s2, (void*)L.q13k, (void*)L.q2k,
                  (void*)L.s2k, (void*)L.s13k}) {
    if (!p) continue;
    for (auto it = layer->allocations.begin(); it != layer->allocations.end(); ++it)
      if (*it == p) {
        layer->allocations.erase(it);
        break;
      }
    (void)hipFree(p);
  }
  for (void* p : fresh) layer->allocations.push_back(p);
  layer->bytes += 2 * n13 + 2 * (n13 / 32 * 4) + 2 * n2 + 2 * (n2 / 32 * 4);
  L.q13 = static_cast<const int8_t*>(q13);
  L.s13 = static_cast<const float*>(s13);
  L.q2 = static_cast<const int8_t*>(q2);
  L.s2 = static_cast<const float*>(s2);
  L.q13k = static_cast<const int8_t*>(q13k);
  L.q2k = static_cast<const int8_t*>(q2k);
  L.s2k = static_cast<const float*>(s2k);
  L.s13k = static_cast<const float*>(s13k);
  L.quant_mode = mode;
  layer->quant_mode = mode;
  return UOCR_OK;
}

const char* uocr_moe_layer_precision(const uocr_moe_layer* layer) {
  if (!layer) return "";
  switch (layer->quant_mode) {
    case UOCR_QUANT_WEIGHTS_ONLY:
      return "int8_weights_fp32";
    case UOCR_QUANT_DYNAMIC_ACTIVATIONS:
      return "int8_weights_dynamic_activations";
    default:
      return "bf16_weights_fp32";
  }
}

size_t uocr_moe_layer_device_bytes(const uocr_moe_layer* layer) { return layer ? layer->bytes : 0; }

void uocr_moe_layer_destroy(uocr_moe_layer* layer) {
  if (!layer) return;
  (void)hipSetDevice(layer->device);
  for (void* p : layer->allocations) (void)hipFree(p);
  delete layer;
}

int uocr_moe_forward_async(uocr_gpu_ctx* ctx, const uocr_moe_layer* layer, const float* x,
                           size_t T, float* y, uint32_t flags, const uocr_moe_trace* trace) {
  if (!ctx || !layer) return fail(UOCR_ERR_SHAPE, "null handle");
  if (T == 0) return UOCR_OK;
  if (!x || !y) return fail(UOCR_ERR_SHAPE, "null activation pointer");
  if (layer->device != ctx->device) return fail(UOCR_ERR_SHAPE, "layer lives on another device");
  if (T > max_tokens(layer->cfg))
    return fail(UOCR_ERR_RESOURCE, "token count too large for one forward (%zu > %zu)", T,
                max_tokens(layer->cfg));
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  return enqueue_experts(exec_of(ctx), layer, x, T, nullptr, y, flags, trace, false);
}

int uocr_moe_forward(uocr_gpu_ctx* ctx, const uocr_moe_layer* layer, const float* x, size_t T,
                     float* y, uint32_t flags, const uocr_moe_trace* trace) {
  int r = uocr_moe_forward_async(ctx, layer, x, T, y, flags, trace);
  if (r) return r;
  return read_and_clear_error(ctx);
}

int uocr_moe_forward_static(const uocr_moe_layer* layer, const float* x, size_t T, float* y,
                            uint32_t flags, int32_t* device_status, void* stream) {
  if (!layer) return fail(UOCR_ERR_SHAPE, "null handle");
  if (T == 0) return UOCR_OK;
  if (!x || !y) return fail(UOCR_ERR_SHAPE, "null activation pointer");
  if (T > max_tokens(layer->cfg))
    return fail(UOCR_ERR_RESOURCE, "token count too large for one forward (%zu > %zu)", T,
                max_tokens(layer->cfg));
  const size_t need = plan_scratch(layer->cfg, T).total;
  const size_t have = (size_t)UOCR_STATIC_SCRATCH_BYTES - kStaticFlagBytes;
  if (need > have)
    return fail(UOCR_ERR_RESOURCE,
                "a forward of %zu tokens needs %zu scratch bytes; the static scratch holds %zu", T,
                need, have);
  HIP_TRY(hipSetDevice(layer->device), "set device");
  std::call_once(g_attr_once, [] {
    uocr::gemv_init_attributes();
    uocr::mfma_init_attributes();
  });
  char* base = nullptr;
  if (int r = static_scratch_of(layer->device, &base)) return r;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int* err = device_status ? reinterpret_cast<int*>(device_status) : reinterpret_cast<int*>(base);
  // A fill kernel, not a memset, so that graph capture records a kernel node.
  int* sync = reinterpret_cast<int*>(base + kSyncOffset);
  float* part = reinterpret_cast<float*>(base + kPartOffset);
  hipLaunchKernelGGL(clear_flag_kernel, dim3(uocr::kDecodePartBytes / 16 / 256), dim3(256), 0, st,
                     err, sync, part);
  Exec ex{base + kStaticFlagBytes, have, st, err, nullptr};
  ex.sync = sync;
  ex.part = part;
  return enqueue_experts(ex, layer, x, T, nullptr, y, flags, nullptr, false);
}

int uocr_moe_block_forward_async(uocr_gpu_ctx* ctx, const uocr_moe_layer* const* layers,
                                 size_t n_layers, const float* x, size_t T, float* y,
                                 uint32_t flags) {
  if (!ctx || (!layers && n_layers)) return fail(UOCR_ERR_SHAPE, "null handle");
  if (T == 0 || n_layers == 0) return UOCR_OK;
  if (!x || !y) return fail(UOCR_ERR_SHAPE, "null activation pointer");
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  for (size_t l = 0; l < n_layers; l++) {
    if (!layers[l]) return fail(UOCR_ERR_SHAPE, "null layer %zu", l);
    // Every layer reads and writes the caller's [T, H] rows.
    if (layers[l]->cfg.hidden_size != layers[0]->cfg.hidden_size)
      return fail(UOCR_ERR_SHAPE, "layer %zu hidden size differs from layer 0", l);
    if (layers[l]->device != ctx->device)
      return fail(UOCR_ERR_SHAPE, "layer %zu lives on another device", l);
    if (T > max_tokens(layers[l]->cfg))
      return fail(UOCR_ERR_RESOURCE, "token count too large for one forward (%zu > %zu)", T,
                  max_tokens(layers[l]->cfg));
    if (!layers[l]->dev.norm_w) return fail(UOCR_ERR_FORMAT, "layer %zu has no norm weight", l);
    if (plan_scratch(layers[l]->cfg, T).total > ctx->scratch_limit)
      return fail(UOCR_ERR_RESOURCE, "operation exceeds scratch limit");
  }
  // Layer l's RMSNorm (and the bf16 planes of its output when layer l uses
  // the MFMA engine) runs fused into layer l - 1's combine when both layers
  // have the same scratch layout and the combine is not the decode
  // engine's; otherwise as a kernel of its own.
  auto norm_of = [&](size_t l, const Scratch& S) {
    const uocr_moe_layer* layer = layers[l];
    uocr::RowNorm nn;
    nn.w = layer->dev.norm_w;
    nn.eps = layer->dev.eps;
    nn.out = S.xn;
    if (choose_engine(layer, T, flags) == Engine::Mfma && uocr::row_norm_fusable(layer->dev.H))
      input_planes(S, layer->dev, T, flags, &nn.hi, &nn.lo);
    return nn;
  };
  const float* cur = x;
  bool normed = false;  // layer l's norm already ran (fused)
  for (size_t l = 0; l < n_layers; l++) {
    const uocr_moe_layer* layer = layers[l];
    const ScratchPlan plan = plan_scratch(layer->cfg, T);
    Scratch S = carve(exec_of(ctx), plan);
    const uocr::RowNorm nn = norm_of(l, S);
    if (!normed) {
      phase_begin(ctx, kNorm);
      uocr::launch_rms_norm(cur, (int)T, layer->dev.H, nn, S.err, ctx->stream);
      phase_end(ctx);
    }
    uocr::RowNorm next;
    bool want = false;
    if (l + 1 < n_layers && uocr::row_norm_fusable(layer->dev.H)) {
      // Same scratch layout: the shapes plan_scratch reads.
      const uocr_moe_config &a = layer->cfg, &b = layers[l + 1]->cfg;
      if (a.hidden_size == b.hidden_size && a.moe_intermediate_size == b.moe_intermediate_size &&
          a.n_routed_experts == b.n_routed_experts && a.n_shared_experts == b.n_shared_experts &&
          a.num_experts_per_tok == b.num_experts_per_tok) {
        next = norm_of(l + 1, S);
        want = true;
      }
    }
    bool fused = false;
    int r = enqueue_experts(exec_of(ctx), layer, S.xn, T, cur, y, flags, nullptr, true,
                            nn.hi != nullptr, want ? &next : nullptr, &fused);
    if (r) return r;
    normed = fused;
    cur = y;
  }
  return UOCR_OK;
}

int uocr_moe_block_forward(uocr_gpu_ctx* ctx, const uocr_moe_layer* const* layers,
                           size_t n_layers, const float* x, size_t T, float* y, uint32_t flags) {
  int r = uocr_moe_block_forward_async(ctx, layers, n_layers, x, T, y, flags);
  if (r) return r;
  return read_and_clear_error(ctx);
}

int uocr_route(uocr_gpu_ctx* ctx, const float* logits, size_t T, size_t n, size_t count,
               int normalize, float scale, int32_t* ids, float* weights) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  // moe::route argument rules (src/decoder/moe.rs:13-15).
  if (count == 0 || count > n || !std::isfinite(scale) || scale <= 0.f)
    return fail(UOCR_ERR_SHAPE, "invalid expert routing");
  if (n > 64 || count > 64) return fail(UOCR_ERR_UNSUPPORTED, "GPU routing supports <= 64 logits");
  if (T == 0) return UOCR_OK;
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  uocr::launch_topk(logits, (int)T, (int)n, (int)count, normalize, scale, ids, weights, ctx->err,
                    ctx->stream);
  HIP_TRY(hipGetLastError(), "kernel launch");
  return read_and_clear_error(ctx);
}

int uocr_linear_bf16(uocr_gpu_ctx* ctx, const float* x, size_t m, size_t k, const uint16_t* w,
                     size_t n, float* y) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  if (k == 0 || n == 0) return fail(UOCR_ERR_SHAPE, "linear weight must be [out,in]");
  if (m == 0) return UOCR_OK;
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  uocr::launch_linear_bf16(x, (int)m, (int)k, w, (int)n, y, ctx->stream);
  HIP_TRY(hipGetLastError(), "kernel launch");
  return read_and_clear_error(ctx);
}

int uocr_int8_linear(uocr_gpu_ctx* ctx, const int8_t* q, const float* scales, size_t rows,
                     size_t cols, const float* x, size_t batch, float* y) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  if (rows == 0 || cols == 0) return fail(UOCR_ERR_SHAPE, "INT8 matrix storage");
  if (batch == 0) return UOCR_OK;
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  uocr::launch_int8_linear(q, scales, (int)rows, (int)cols, x, (int)batch, y, ctx->stream);
  HIP_TRY(hipGetLastError(), "kernel launch");
  return read_and_clear_error(ctx);
}

int uocr_int8_linear_dynamic(uocr_gpu_ctx* ctx, const int8_t* q, const float* scales,
                             size_t rows, size_t cols, const float* x, float* y,
                             int32_t* block_sums) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  if (rows == 0 || cols == 0) return fail(UOCR_ERR_SHAPE, "INT8 matrix storage");
  const size_t blocks = (cols + 31) / 32;
  // src/cpu/quantized.rs:162-168 scratch: the quantised row and its scales.
  if (align256(cols) + blocks * 4 > ctx->scratch_limit)
    return fail(UOCR_ERR_RESOURCE, "operation exceeds scratch limit");
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  int8_t* xq = reinterpret_cast<int8_t*>(ctx->scratch);
  float* xs = reinterpret_cast<float*>(ctx->scratch + align256(cols));
  uocr::launch_int8_dynamic(q, scales, (int)rows, (int)cols, x, y, block_sums, xq, xs, ctx->err,
                            ctx->stream);
  HIP_TRY(hipGetLastError(), "kernel launch");
  return read_and_clear_error(ctx);
}

int uocr_rms_norm(uocr_gpu_ctx* ctx, const float* x, size_t rows, size_t width,
                  const float* weight, float eps, float* out) {
  if (!ctx) return fail(UOCR_ERR_SHAPE, "null context");
  if (width == 0 || !std::isfinite(eps) || eps <= 0.f)
    return fail(UOCR_ERR_SHAPE, "invalid normalization parameters");
  if (rows == 0) return UOCR_OK;
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  uocr::RowNorm nn;
  nn.w = weight;
  nn.eps = eps;
  nn.out = out;
  uocr::launch_rms_norm(x, (int)rows, (int)width, nn, ctx->err, ctx->stream);
  HIP_TRY(hipGetLastError(), "kernel launch");
  return read_and_clear_error(ctx);
}


// ------------------------------------------------- vocabulary projection

int uocr_lm_head_create(uocr_gpu_ctx* ctx, const uocr_lm_head_weights* w, uocr_memory where,
                        uocr_lm_head** out) {
  if (!ctx || !w || !out) return fail(UOCR_ERR_SHAPE, "null handle");
  *out = nullptr;
  const size_t V = w->vocab_size, H = w->hidden_size;
  if (V == 0 || H == 0) return fail(UOCR_ERR_SHAPE, "lm_head must be [vocab, hidden]");
  if (V > (size_t)INT32_MAX / 2 || H > 65536) return fail(UOCR_ERR_UNSUPPORTED, "lm_head too large");
  if (!w->norm_weight) return fail(UOCR_ERR_FORMAT, "missing model.norm.weight");
  if (!std::isfinite(w->rms_norm_eps) || w->rms_norm_eps <= 0.f)
    return fail(UOCR_ERR_SHAPE, "invalid normalization parameters");
  const bool quant = w->q != nullptr;
  if (quant) {
    if (w->quant_mode != UOCR_QUANT_WEIGHTS_ONLY && w->quant_mode != UOCR_QUANT_DYNAMIC_ACTIVATIONS)
      return fail(UOCR_ERR_SHAPE, "an INT8 lm_head needs a quantization mode");
    if (!w->scales) return fail(UOCR_ERR_FORMAT, "missing lm_head.weight.q8_scales");
    if (H % 32) return fail(UOCR_ERR_SHAPE, "INT8 lm_head width must be a multiple of 32");
  } else {
    if (w->quant_mode != UOCR_QUANT_NONE)
      return fail(UOCR_ERR_FORMAT, "quantized lm_head without INT8 weights");
    if (!w->weight) return fail(UOCR_ERR_FORMAT, "missing lm_head.weight");
  }
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  auto* head = new uocr_lm_head();
  head->device = ctx->device;
  head->view.V = (int)V;
  head->view.H = (int)H;
  head->view.eps = w->rms_norm_eps;
  head->view.kind = !quant ? 0 : (w->quant_mode == UOCR_QUANT_DYNAMIC_ACTIVATIONS ? 2 : 1);
  auto finish = [&](int status) {
    if (status) uocr_lm_head_destroy(head);
    return status;
  };
  auto alloc_copy = [&](const void* src, size_t bytes, void** dst) -> int {
    hipError_t e = hipMalloc(dst, bytes);
    if (e != hipSuccess) return hip_fail(e, "lm_head allocation");
    head->allocations.push_back(*dst);
    head->bytes += bytes;
    if ((e = hipMemcpyAsync(*dst, src, bytes, kind_of(where), ctx->stream)) != hipSuccess)
      return hip_fail(e, "lm_head upload");
    return UOCR_OK;
  };
  void* p = nullptr;
  int r = alloc_copy(w->norm_weight, H * 4, &p);
  if (r) return finish(r);
  head->view.norm_w = static_cast<const float*>(p);
  if (quant) {
    if ((r = alloc_copy(w->q, V * H, &p))) return finish(r);
    head->view.q = static_cast<const int8_t*>(p);
    if ((r = alloc_copy(w->scales, V * (H / 32) * 4, &p))) return finish(r);
    head->view.s = static_cast<const float*>(p);
  } else {
    if ((r = alloc_copy(w->weight, V * H * 2, &p))) return finish(r);
    head->view.w = static_cast<const uint16_t*>(p);
  }
  HIP_TRY(hipStreamSynchronize(ctx->stream), "lm_head upload");
  *out = head;
  return UOCR_OK;
}

int uocr_lm_head_logits_async(uocr_gpu_ctx* ctx, const uocr_lm_head* head, const float* hidden,
                              size_t T, float* logits) {
  if (!ctx || !head) return fail(UOCR_ERR_SHAPE, "null handle");
  if (T == 0 || !hidden) return fail(UOCR_ERR_SHAPE, "missing final hidden state");
  if (!logits) return fail(UOCR_ERR_SHAPE, "null logits");
  if (head->device != ctx->device) return fail(UOCR_ERR_SHAPE, "lm_head lives on another device");
  HIP_TRY(hipSetDevice(ctx->device), "set device");
  const uocr::LmHeadView& v = head->view;
  const float* last = hidden + (T - 1) * (size_t)v.H;
  if (uocr::lm_head_fast(v.H)) {
    uocr::launch_lm_head(last, v, logits, ctx->err, ctx->stream);
  } else {
    // Other widths: the norm into scratch, then the single-matrix operators.
    const size_t blocks = (size_t)v.H / 32;
    if (align256((size_t)v.H * 4) + align256(v.H) + blocks * 4 > ctx->scratch_limit)
      return fail(UOCR_ERR_RESOURCE, "operation exceeds scratch limit");
    float* xn = reinterpret_cast<float*>(ctx->scratch);
    uocr::RowNorm nn;
    nn.w = v.norm_w;
    nn.eps = v.eps;
    nn.out = xn;
    uocr::launch_rms_norm(last, 1, v.H, nn, ctx->err, ctx->stream);
    if (v.kind == 0) {
      uocr::launch_linear_bf16(xn, 1, v.H, v.w, v.V, logits, ctx->stream);
    } else if (v.kind == 1) {
      uocr::launch_int8_linear(v.q, v.s, v.V, v.H, xn, 1, logits, ctx->stream);
    } else {
      int8_t* xq = reinterpret_cast<int8_t*>(ctx->scratch + align256((size_t)v.H * 4));
      float* xs = reinterpret_cast<float*>(ctx->scratch + align256((size_t)v.H * 4) + align256(v.H));
      uocr::launch_int8_dynamic(v.q, v.s, v.V, v.H, xn, logits, nullptr, xq, xs, ctx->err,
                                ctx->stream);
    }
  }
  HIP_TRY(hipGetLastError(), "kernel launch");
  return UOCR_OK;
}

int uocr_lm_head_logits(uocr_gpu_ctx* ctx, const uocr_lm_head* head, const float* hidden,
                        size_t T, float* logits) {
  int r = uocr_lm_head_logits_async(ctx, head, hidden, T, logits);
  if (r) return r;
  return read_and_clear_error(ctx);
}

const char* uocr_lm_head_precision(const uocr_lm_head* head) {
  if (!head) return "";
  return head->view.kind == 0   ? "bf16_weights_fp32"
         : head->view.kind == 1 ? "int8_weights_fp32"
                                : "int8_weights_dynamic_activations";
}

size_t uocr_lm_head_device_bytes(const uocr_lm_head* head) { return head ? head->bytes : 0; }

void uocr_lm_head_destroy(uocr_lm_head* head) {
  if (!head) return;
  if (hipSetDevice(head->device) == hipSuccess)
    for (void* p : head->allocations) (void)hipFree(p);
  delete head;
}

}  // extern "C"
