/*
 * uocr_moe — MI355X (gfx950) MoE feed-forward path of the Unlimited-OCR
 * decoder behind a plain C ABI.
 *
 * The reference is the Rust crate `uocr`; this library replaces the body of
 * `Decoder::experts` (src/decoder/mod.rs:124-220) and the CPU kernels it
 * calls, and adds the GPU counterparts of the operator entry points the
 * reference tests exercise. All pointers are plain host or device pointers
 * with explicit sizes; no torch or Rust types cross the boundary.
 *
 * Status codes follow the order of the reference's OcrError variants
 * (src/error.rs:1-19): Io, Json, Format, Shape, Unsupported, Resource,
 * Numerical. A failing call leaves its outputs unspecified, like an Err.
 */
#ifndef UOCR_MOE_H
#define UOCR_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum uocr_status {
  UOCR_OK = 0,
  UOCR_ERR_IO = 1,
  UOCR_ERR_JSON = 2,
  UOCR_ERR_FORMAT = 3,
  UOCR_ERR_SHAPE = 4,
  UOCR_ERR_UNSUPPORTED = 5,
  UOCR_ERR_RESOURCE = 6,
  UOCR_ERR_NUMERICAL = 7,
} uocr_status;

/* QuantizationMode (src/cpu/quantized.rs:242-247), plus "no overlay". */
typedef enum uocr_quant_mode {
  UOCR_QUANT_NONE = 0,                /* BF16 weights, FP32 activations */
  UOCR_QUANT_WEIGHTS_ONLY = 1,        /* QuantizationMode::WeightsOnly */
  UOCR_QUANT_DYNAMIC_ACTIVATIONS = 2, /* QuantizationMode::DynamicActivations */
} uocr_quant_mode;

/* Backend (src/cpu/mod.rs:10-16) with the GPU variant this library adds. */
typedef enum uocr_backend {
  UOCR_BACKEND_SCALAR = 0,
  UOCR_BACKEND_NEON = 1,
  UOCR_BACKEND_ACCELERATE = 2,
  UOCR_BACKEND_AUTO = 3,
  UOCR_BACKEND_GPU = 4,
} uocr_backend;

/* Where the pointers handed to uocr_moe_layer_create live. */
typedef enum uocr_memory {
  UOCR_MEMORY_HOST = 0,
  UOCR_MEMORY_DEVICE = 1,
} uocr_memory;

/* Forward flags. The multi-row MFMA path rounds its FP32 activations to
 * bf16 operands: FP32_CLASS splits each activation into two bf16 terms
 * (relative error ~2^-17, the 1e-3 tolerance class); BF16 uses one term
 * (the 2e-2 class). Decode GEMV paths always compute in FP32. */
#define UOCR_FLAG_FP32_CLASS 0u
#define UOCR_FLAG_BF16_ACTIVATIONS 1u
/* Force one expert engine, for tests: 0 = choose by token count. */
#define UOCR_FLAG_FORCE_GEMV 2u
#define UOCR_FLAG_FORCE_MFMA 4u
/* Opt-in extension for DynamicActivations layers (else Unsupported): every
 * expert group, whatever its row count, computes as
 * Int8Matrix::linear_dynamic_int8 row by row (activations quantised per
 * 32-block, int8 x int8 products with exact int32 block sums on the int8
 * MFMA). The reference does this for single-row groups only
 * (src/decoder/mod.rs:103-104), so for multi-row groups the results differ
 * from it by the activation rounding (the W8A8 tolerance class). */
#define UOCR_FLAG_INT8_MFMA 8u

/* The MoE fields of ModelConfig (src/model/config.rs:35-54). */
typedef struct uocr_moe_config {
  uint32_t hidden_size;           /* 1280 */
  uint32_t moe_intermediate_size; /* 896 */
  uint32_t n_routed_experts;      /* 64 */
  uint32_t n_shared_experts;      /* 2 */
  uint32_t num_experts_per_tok;   /* 6 */
  uint32_t norm_topk_prob;        /* bool */
  float routed_scaling_factor;    /* 1.0 */
  float rms_norm_eps;             /* 1e-6 */
} uocr_moe_config;

/* BF16 checkpoint tensors of one MoE layer, row-major [out, in] as stored
 * under model.layers.N.mlp.* (src/decoder/mod.rs:58-80); raw bf16 bits.
 * E = n_routed_experts, I = moe_intermediate_size, S = I * n_shared_experts,
 * H = hidden_size. norm_weight (post_attention_layernorm) may be NULL unless
 * uocr_moe_block_forward is used. */
typedef struct uocr_moe_bf16_weights {
  const uint16_t* router;      /* mlp.gate.weight               [E,H]   */
  const uint16_t* expert_gate; /* mlp.experts.*.gate_proj       [E,I,H] */
  const uint16_t* expert_up;   /* mlp.experts.*.up_proj         [E,I,H] */
  const uint16_t* expert_down; /* mlp.experts.*.down_proj       [E,H,I] */
  const uint16_t* shared_gate; /* mlp.shared_experts.gate_proj  [S,H]   */
  const uint16_t* shared_up;   /* mlp.shared_experts.up_proj    [S,H]   */
  const uint16_t* shared_down; /* mlp.shared_experts.down_proj  [H,S]   */
  const uint16_t* norm_weight; /* post_attention_layernorm      [H]     */
} uocr_moe_bf16_weights;

/* INT8 block-32 overlay matrices (src/cpu/quantized.rs:9-42, 239-369):
 * int8 [rows, cols] and f32 scales [rows, cols/32]. The router is never
 * part of the overlay. */
typedef struct uocr_moe_int8_weights {
  const int8_t* expert_gate;
  const float* expert_gate_scales;
  const int8_t* expert_up;
  const float* expert_up_scales;
  const int8_t* expert_down;
  const float* expert_down_scales;
  const int8_t* shared_gate;
  const float* shared_gate_scales;
  const int8_t* shared_up;
  const float* shared_up_scales;
  const int8_t* shared_down;
  const float* shared_down_scales;
} uocr_moe_int8_weights;

/* Optional trace of the W8A8 projections (DynamicActivations): the exact
 * int32 block sums of Int8Matrix::linear_dynamic_int8
 * (src/cpu/quantized.rs:190-198, sum over one 32-block of q_w * q_x) for
 * every row a single-row group projects, and the FP32 hidden row
 * (silu(gate) * up) that entered its down projection. Routed entries are
 * indexed by dispatched position p (expert_offsets order):
 *   gateup_sums [T*k][2*I][H/32]  rows 0..I-1 gate_proj, I..2I-1 up_proj
 *   down_sums   [T*k][H][I/32]
 *   hidden      [T*k][I]
 * Positions of multi-row groups are left untouched (under
 * UOCR_FLAG_INT8_MFMA every group computes this way, so every position is
 * written). The shared expert is a single-row group only when T == 1:
 *   shared_gateup_sums [2*S][H/32], shared_down_sums [H][S/32],
 *   shared_hidden [S].
 * Device pointers; NULL members are skipped. */
typedef struct uocr_w8a8_trace {
  int32_t* gateup_sums;
  int32_t* down_sums;
  float* hidden;
  int32_t* shared_gateup_sums;
  int32_t* shared_down_sums;
  float* shared_hidden;
} uocr_w8a8_trace;

/* Optional per-forward trace, device pointers; NULL members are skipped.
 * Routing order is route()'s: probability descending, id ascending.
 *
 * decode_stamps (an instrument with no counterpart in the reference): for a
 * forward on the one-token engine, the device's 100 MHz real-time counter
 * at the phase boundaries of every workgroup of its launch, as
 * [UOCR_DECODE_STAMP_ROWS(E, S, k, I, H)][8] uint64 (S = the shared width,
 * I * n_shared_experts). Rows in launch order and their stamps:
 *   ceil(E/8) router-logit workgroups: 0 start, 1 logits stored, 2 stores
 *     complete, 3 counted in;
 *   S/32 shared gate/up workgroups: 0 start, 3 rows dotted, 4 counted in
 *     (BF16 layers) or down partials stored (INT8 overlays);
 *   k*I/32 routed gate/up workgroups: 0 start, 1 input staged (INT8
 *     overlays: and the workgroup's copy of the logits in), 2 experts
 *     selected, 3 rows dotted, 4 as the shared ones;
 *   H/8 output workgroups. BF16 layers (down workgroups): 0 start, 1
 *     experts selected, 3 every hidden value ready, 4 rows dotted, 5 output
 *     written. INT8 overlays (combine workgroups, which read the gate/up
 *     workgroups' down partials): 0 start, 1 experts selected, 2 probe
 *     partial in, 3 every partial read, 4 partials summed, 5 output written.
 * Other stamps are left untouched. Other engines ignore the member. */
#define UOCR_DECODE_STAMPS 8
#define UOCR_DECODE_STAMP_ROWS(E, S, k, I, H) \
  (((E) + 7) / 8 + (S) / 32 + (k) * ((I) / 32) + (H) / 8)
typedef struct uocr_moe_trace {
  float* logits;           /* [T,E] router logits */
  int32_t* topk_ids;       /* [T,k] */
  float* topk_weights;     /* [T,k] */
  int32_t* expert_offsets; /* [E+1] start of each expert's assignments */
  int32_t* perm_rows;      /* [T*k] token row of each assignment, expert-major */
  float* perm_weights;     /* [T*k] routing weight of each assignment */
  const uocr_w8a8_trace* w8a8; /* W8A8 block sums (NULL: none) */
  uint64_t* decode_stamps; /* one-token engine timeline (NULL: none) */
} uocr_moe_trace;

typedef struct uocr_gpu_ctx uocr_gpu_ctx;
typedef struct uocr_moe_layer uocr_moe_layer;

/* ---------------------------------------------------------------- context */

/* CpuContext::new(Backend, threads, scratch_limit) (src/cpu/mod.rs:26-49),
 * GPU flavour: binds `device`, creates the context's stream and reserves
 * `scratch_limit` bytes of device scratch. 0 bytes -> Resource, like
 * threads == 0 or scratch_limit == 0 in the reference. */
int uocr_gpu_ctx_create(int device, size_t scratch_limit, uocr_gpu_ctx** out);
void uocr_gpu_ctx_destroy(uocr_gpu_ctx* ctx);
/* The stream work is enqueued on (a hipStream_t). */
void* uocr_gpu_ctx_stream(uocr_gpu_ctx* ctx);
/* Waits for the context's stream and reports errors raised on the device
 * (non-finite routing, normalisation or activation quantisation inputs ->
 * Numerical), then clears them. */
int uocr_gpu_ctx_synchronize(uocr_gpu_ctx* ctx);
/* Message of the last failure on this thread (ctx may be NULL). */
const char* uocr_last_error(const uocr_gpu_ctx* ctx);
/* Phase timing with HIP events on the context stream (the GPU side of the
 * reference's per-phase Timings, src/model/mod.rs:36-45). Bit i of
 * phase_mask brackets every launch of phase i with events; totals
 * accumulate until read. Phases, in bit order: router, topk, dispatch,
 * split, gateup, down, combine, norm, decode (the one-token engine's
 * single launch). 0 disables timing. */
typedef struct uocr_phase_time {
  const char* name;
  uint64_t launches;
  double total_ms;
} uocr_phase_time;
int uocr_gpu_ctx_set_timing(uocr_gpu_ctx* ctx, uint32_t phase_mask);
/* Synchronises, then copies up to `cap` phase totals (all phases when cap
 * allows) and resets them. *count receives the number of phases. */
int uocr_gpu_ctx_timings(uocr_gpu_ctx* ctx, uocr_phase_time* out, size_t cap, size_t* count);
/* No counterpart in the reference: a diagnostic control for the one-token
 * engine, whose single launch has workgroups wait for others (bounded
 * polls; a wait that reaches its bound raises Resource and the launch
 * still ends). polls < 0 restores the default bound (~100 ms); 0 makes
 * every wait that is not already satisfied give up at once, which is how
 * the tests drive that error path. */
int uocr_gpu_ctx_set_wait_limit(uocr_gpu_ctx* ctx, int polls);
/* Bytes of scratch a forward of T tokens needs (CpuContext::check_elements,
 * src/cpu/mod.rs:73-78); forwards above the context's limit fail with
 * Resource. */
size_t uocr_moe_scratch_bytes(const uocr_moe_config* cfg, size_t T);
/* Most tokens one forward of this configuration accepts (the device
 * engines address activation planes with 32-bit byte offsets); more ->
 * Resource. No counterpart in the reference, whose tensors are host
 * vectors. */
size_t uocr_moe_max_tokens(const uocr_moe_config* cfg);

/* ------------------------------------------------------------------ layer */

/* Decoder::new shape rules for one MoE layer (src/decoder/mod.rs:32-88) and
 * ModelConfig validation (src/model/config.rs:74-115) for the MoE fields;
 * uploads and repacks the BF16 weights once. The GPU layer supports
 * hidden_size and moe_intermediate_size that are multiples of 64,
 * n_routed_experts <= 64 and num_experts_per_tok <= 8 (else Unsupported). */
int uocr_moe_layer_create(uocr_gpu_ctx* ctx, const uocr_moe_config* cfg,
                          const uocr_moe_bf16_weights* weights, uocr_memory where,
                          uocr_moe_layer** out);
/* Model::load_with_quantization overlay step (src/model/mod.rs:82-109,
 * src/cpu/quantized.rs:306-366): validates and uploads the INT8 matrices and
 * selects the mode. DynamicActivations without an overlay -> Format. */
int uocr_moe_layer_attach_int8(uocr_gpu_ctx* ctx, uocr_moe_layer* layer,
                               const uocr_moe_int8_weights* weights, uocr_memory where,
                               uocr_quant_mode mode);
/* Model::precision labels (src/model/mod.rs:65-73). */
const char* uocr_moe_layer_precision(const uocr_moe_layer* layer);
/* Device bytes held by the layer's weights. */
size_t uocr_moe_layer_device_bytes(const uocr_moe_layer* layer);
void uocr_moe_layer_destroy(uocr_moe_layer* layer);

/* ---------------------------------------------------------------- forward */

/* Decoder::experts (src/decoder/mod.rs:124-220): y[T,H] = shared(x) +
 * sum over each row's top-k experts, ascending id, of p * expert(x).
 * x and y are device pointers (FP32 row-major [T,H]). Enqueued on the
 * context stream; the call returns once the work is queued. Device-side
 * errors surface at uocr_gpu_ctx_synchronize. T == 0 is a no-op. */
int uocr_moe_forward_async(uocr_gpu_ctx* ctx, const uocr_moe_layer* layer, const float* x,
                           size_t T, float* y, uint32_t flags, const uocr_moe_trace* trace);
/* The same, then synchronize: errors are reported by this call. */
int uocr_moe_forward(uocr_gpu_ctx* ctx, const uocr_moe_layer* layer, const float* x, size_t T,
                     float* y, uint32_t flags, const uocr_moe_trace* trace);
/* Allocation-free variant of uocr_moe_forward_async. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). Same engines and results as uocr_moe_forward_async, but its
 * scratch is a static device array of UOCR_STATIC_SCRATCH_BYTES per GPU
 * (held until the process ends) instead of a context's reservation, and it
 * calls no allocating routine. Its first UOCR_STATIC_RESERVED_BYTES hold
 * the device flag and the one-token engines' synchronisation words, down
 * partials and logit copies (a fill kernel, not a memset, resets them at every call);
 * forwards whose uocr_moe_scratch_bytes exceeds UOCR_STATIC_SCRATCH_BYTES -
 * UOCR_STATIC_RESERVED_BYTES fail with Resource (at the model shape: up to
 * 126 tokens). Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU race, so serialise them (one
 * stream, or events). Enqueued on `stream` (a hipStream_t; NULL: the null
 * stream) and returns once queued. Device-side errors (non-finite
 * routing, normalisation or W8A8 inputs: Numerical; a one-token launch
 * whose workgroups did not all run: Resource) are written as a status code
 * to *device_status (a device int32 the call first clears; NULL: an
 * internal flag nobody reads). No trace, no phase timers. */
#define UOCR_STATIC_SCRATCH_BYTES (20u << 20)
#define UOCR_STATIC_RESERVED_BYTES (256u + (64u << 10) + (328u << 13))
int uocr_moe_forward_static(const uocr_moe_layer* layer, const float* x, size_t T, float* y,
                            uint32_t flags, int32_t* device_status, void* stream);
/* The post-attention half of Decoder::layer (src/decoder/mod.rs:351-363)
 * over a stack of MoE layers: x <- x + experts(rms_norm(x, norm_weight)),
 * layer after layer. x and y are device [T,H]; y may equal x. Synchronous. */
int uocr_moe_block_forward(uocr_gpu_ctx* ctx, const uocr_moe_layer* const* layers,
                           size_t n_layers, const float* x, size_t T, float* y, uint32_t flags);
int uocr_moe_block_forward_async(uocr_gpu_ctx* ctx, const uocr_moe_layer* const* layers,
                                 size_t n_layers, const float* x, size_t T, float* y,
                                 uint32_t flags);

/* ------------------------------------------------------------- operators */
/* Device counterparts of the reference's CPU operators, on device pointers,
 * synchronous. They back the operator-level parity tests. */

/* moe::route over T rows of n logits (src/decoder/moe.rs:7-30). */
int uocr_route(uocr_gpu_ctx* ctx, const float* logits, size_t T, size_t n, size_t count,
               int normalize, float scale, int32_t* ids, float* weights);
/* ops::linear_weight with a BF16 [n,k] matrix and no bias
 * (src/cpu/ops.rs:62-133): y[m,n] = x[m,k] . w^T in FP32. */
int uocr_linear_bf16(uocr_gpu_ctx* ctx, const float* x, size_t m, size_t k, const uint16_t* w,
                     size_t n, float* y);
/* Int8Matrix::linear (src/cpu/quantized.rs:99-150). */
int uocr_int8_linear(uocr_gpu_ctx* ctx, const int8_t* q, const float* scales, size_t rows,
                     size_t cols, const float* x, size_t batch, float* y);
/* Int8Matrix::linear_dynamic_int8 (src/cpu/quantized.rs:155-236): one input
 * row. block_sums (optional, [rows, cols/32]) receives the exact i32
 * per-block accumulators. */
int uocr_int8_linear_dynamic(uocr_gpu_ctx* ctx, const int8_t* q, const float* scales,
                             size_t rows, size_t cols, const float* x, float* y,
                             int32_t* block_sums);
/* ops::rms_norm (src/cpu/ops.rs:362-423), rows x width. */
int uocr_rms_norm(uocr_gpu_ctx* ctx, const float* x, size_t rows, size_t width,
                  const float* weight, float eps, float* out);

/* ------------------------------------------------- vocabulary projection */
/* Decoder::logits (src/decoder/mod.rs:367-379): the last hidden row,
 * RMSNorm with model.norm.weight, then Decoder::projection (:99-112) with
 * lm_head.weight — BF16, or the INT8 overlay's lm_head.weight
 * (src/cpu/quantized.rs:267-269): weight-only, or W8A8 under
 * DynamicActivations (the projected row is a single row). */
typedef struct uocr_lm_head uocr_lm_head;
typedef struct uocr_lm_head_weights {
  uint32_t vocab_size;   /* V, rows of lm_head.weight */
  uint32_t hidden_size;  /* H */
  float rms_norm_eps;
  const float* norm_weight;  /* model.norm.weight widened to f32, [H] */
  const uint16_t* weight;    /* lm_head.weight bf16 bits [V, H]; may be NULL with q */
  const int8_t* q;           /* overlay lm_head.weight [V, H], or NULL */
  const float* scales;       /* its .q8_scales [V, H/32] */
  uocr_quant_mode quant_mode; /* UOCR_QUANT_NONE when q is NULL */
} uocr_lm_head_weights;
int uocr_lm_head_create(uocr_gpu_ctx* ctx, const uocr_lm_head_weights* w, uocr_memory where,
                        uocr_lm_head** out);
/* logits[V] of hidden[T, H] (device pointers): its last row. T == 0 ->
 * Shape ("missing final hidden state"); non-finite row -> Numerical. */
int uocr_lm_head_logits(uocr_gpu_ctx* ctx, const uocr_lm_head* head, const float* hidden,
                        size_t T, float* logits);
int uocr_lm_head_logits_async(uocr_gpu_ctx* ctx, const uocr_lm_head* head, const float* hidden,
                              size_t T, float* logits);
/* "bf16_weights_fp32", "int8_weights_fp32", "int8_weights_dynamic_activations". */
const char* uocr_lm_head_precision(const uocr_lm_head* head);
size_t uocr_lm_head_device_bytes(const uocr_lm_head* head);
void uocr_lm_head_destroy(uocr_lm_head* head);

/* ---------------------------------------------------- checkpoint files */
/* The model-directory side of Model::load_with_quantization; the C++ form
 * of each is in uocr.hpp. */

/* Safetensors dtypes (DType, src/checkpoint.rs:14-21). */
typedef enum uocr_dtype {
  UOCR_DTYPE_BF16 = 0,
  UOCR_DTYPE_F16 = 1,
  UOCR_DTYPE_F32 = 2,
  UOCR_DTYPE_I64 = 3,
  UOCR_DTYPE_I8 = 4,
} uocr_dtype;

typedef struct uocr_checkpoint uocr_checkpoint;
/* Checkpoint::open (src/checkpoint.rs:114-178): memory-maps a safetensors
 * file and validates its header: < 8 bytes, a header over 100 MB, a
 * truncated header, size overflow, bad offsets, gaps, overlaps or trailing
 * payload -> Format; malformed header JSON -> Json; unreadable file -> Io. */
int uocr_checkpoint_open(const char* path, uocr_checkpoint** out);
void uocr_checkpoint_close(uocr_checkpoint* ckpt);
/* Checkpoint::sha256 (src/checkpoint.rs:183-206): lowercase hex, NUL-ended. */
int uocr_checkpoint_sha256(const uocr_checkpoint* ckpt, char out[65]);
/* Checkpoint::names (src/checkpoint.rs:220-222): sorted; NULL past the end. */
size_t uocr_checkpoint_count(const uocr_checkpoint* ckpt);
const char* uocr_checkpoint_name(const uocr_checkpoint* ckpt, size_t index);
/* Checkpoint::metadata (src/checkpoint.rs:180-182): NULL when absent. */
const char* uocr_checkpoint_metadata(const uocr_checkpoint* ckpt, const char* key);
/* Checkpoint::tensor (src/checkpoint.rs:208-219): dtype, shape (up to
 * max_dims entries) and the mapped bytes; a missing tensor -> Format. */
int uocr_checkpoint_tensor(const uocr_checkpoint* ckpt, const char* name, int* dtype,
                           size_t* shape, size_t max_dims, size_t* ndim, const void** data,
                           size_t* bytes);
/* QuantizedWeights::load (src/cpu/quantized.rs:304-366) without keeping the
 * matrices: manifest (path with ".json"), metadata and SHA-256 binding to
 * `source`, the eligible matrix set and every matrix's storage rules. */
int uocr_overlay_validate(const char* overlay_path, const uocr_checkpoint* source,
                          size_t* matrices);

/* ModelConfig (src/model/config.rs:30-115), the fields this library uses. */
typedef struct uocr_model_config {
  uint32_t hidden_size;
  uint32_t intermediate_size;
  uint32_t moe_intermediate_size;
  uint32_t num_hidden_layers;
  uint32_t num_attention_heads;
  uint32_t num_key_value_heads;
  uint32_t n_routed_experts;
  uint32_t n_shared_experts;
  uint32_t num_experts_per_tok;
  uint32_t first_k_dense_replace;
  uint32_t vocab_size;
  uint32_t norm_topk_prob;
  float routed_scaling_factor;
  float rms_norm_eps;
} uocr_model_config;
/* ModelConfig::load (src/model/config.rs:71-115): unsupported attention or
 * routing -> Unsupported; inconsistent sizes -> Shape; JSON errors -> Json. */
int uocr_config_load(const char* path, uocr_model_config* out);

typedef struct uocr_model uocr_model;
/* Model::load_with_quantization (src/model/mod.rs:82-109) for the MoE
 * layers: config.json and model-00001-of-000001.safetensors in `directory`,
 * the Decoder::new shape rules (src/decoder/mod.rs:32-88), then the overlay
 * (NULL for none). DynamicActivations without an overlay -> Format. Every
 * MoE decoder layer is uploaded to ctx's device. */
int uocr_model_load(uocr_gpu_ctx* ctx, const char* directory, const char* overlay,
                    uocr_quant_mode mode, uocr_model** out);
/* Model::precision (src/model/mod.rs:65-73). */
const char* uocr_model_precision(const uocr_model* model);
/* The layer handle of MoE decoder layer `layer` (NULL for dense layers). */
const uocr_moe_layer* uocr_model_layer(const uocr_model* model, size_t layer);
/* Decoder::experts (src/decoder/mod.rs:124-220) of decoder layer `layer`:
 * y[T,H] from x[T,H], device pointers; synchronous. */
int uocr_model_experts(uocr_gpu_ctx* ctx, const uocr_model* model, size_t layer, const float* x,
                       size_t T, float* y, uint32_t flags);
/* Decoder::logits of a loaded model: logits[vocab_size] of the last row of
 * hidden[T, H] (device pointers); synchronous. */
int uocr_model_logits(uocr_gpu_ctx* ctx, const uocr_model* model, const float* hidden, size_t T,
                      float* logits);
void uocr_model_destroy(uocr_model* model);

#ifdef __cplusplus
}
#endif
#endif
