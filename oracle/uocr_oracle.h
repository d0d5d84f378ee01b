/*
 * CPU oracle for the Unlimited-OCR MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the
 * reported CPU baseline; it is never linked into, loaded by or called from the
 * product library. It restates the reference's x86 scalar branches (no NEON,
 * no Accelerate) with the same sequential reduction orders, separate
 * multiplies and adds (built with -ffp-contract=off) and glibc expf.
 *
 * Every function cites the reference file:line it follows. Status codes follow
 * the order of the reference's OcrError variants (src/error.rs:1-19).
 */
#ifndef UOCR_ORACLE_H
#define UOCR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ORC_OK = 0,
  ORC_IO = 1,
  ORC_JSON = 2,
  ORC_FORMAT = 3,
  ORC_SHAPE = 4,
  ORC_UNSUPPORTED = 5,
  ORC_RESOURCE = 6,
  ORC_NUMERICAL = 7,
};

enum { ORC_QUANT_NONE = 0, ORC_QUANT_WEIGHTS_ONLY = 1, ORC_QUANT_DYNAMIC = 2 };

/* src/checkpoint.rs:79-85: exact widening, bits << 16. */
float orc_bf16_to_f32(uint16_t bits);
/* RNE encode used by the reference's tests (half 2.7.1 bf16::from_f32). */
uint16_t orc_f32_to_bf16(float value);

/* src/cpu/ops.rs:139-187 (Scalar branch). */
int orc_softmax(float* values, size_t n);
/* src/decoder/moe.rs:7-30. ids/weights receive `count` entries. */
int orc_route(const float* logits, size_t n, size_t count, int normalize, float scale,
              int32_t* ids, float* weights);
/* src/cpu/ops.rs:9-59 (scalar triple loop). bias may be NULL. */
int orc_linear(const float* x, size_t m, size_t k, const float* w, size_t n, const float* bias,
               float* y);
/* src/cpu/ops.rs:62-133. BF16 weight [n,k]; m==1 uses the GEMV branch. */
int orc_linear_weight_bf16(const float* x, size_t m, size_t k, const uint16_t* w, size_t n,
                           const float* bias, float* y, int threads);
/* src/cpu/ops.rs:225-229. */
void orc_silu(float* values, size_t n);
/* src/cpu/ops.rs:362-423 (norm with center=false). */
int orc_rms_norm(const float* x, size_t rows, size_t width, const float* weight, float eps,
                 float* out);

/* src/cpu/quantized.rs:18-42 validation of stored INT8 matrices. */
int orc_int8_check(size_t rows, size_t cols, size_t n_weights, size_t n_scales,
                   const float* scales);
/* src/cpu/quantized.rs:43-74. q: [rows*cols], s: [rows*ceil(cols/32)]. */
int orc_int8_quantize(const float* m, size_t rows, size_t cols, int8_t* q, float* s);
/* src/cpu/quantized.rs:75-95. */
void orc_int8_dequantize(const int8_t* q, const float* s, size_t rows, size_t cols, float* out);
/* src/cpu/quantized.rs:99-150. x: [batch, cols] -> y: [batch, rows]. */
int orc_int8_linear(const int8_t* q, const float* s, size_t rows, size_t cols, const float* x,
                    size_t batch, float* y, int threads);
/* src/cpu/quantized.rs:155-236. One input row. block_sums (optional): the
 * i32 per-(row, block) accumulators, [rows * ceil(cols/32)]. */
int orc_int8_linear_dynamic(const int8_t* q, const float* s, size_t rows, size_t cols,
                            const float* x, float* y, int32_t* block_sums, int threads);

/*
 * One MoE layer: router `mlp.gate` + 64 routed experts + the fused shared
 * expert, as Decoder::experts sees them (src/decoder/mod.rs:99-220).
 * Matrices are row-major [out, in] like the checkpoint tensors.
 */
typedef struct orc_moe_layer {
  size_t hidden;      /* H */
  size_t inter;       /* I, moe_intermediate_size */
  size_t shared;      /* S = I * n_shared_experts */
  size_t n_experts;   /* E */
  size_t top_k;       /* k */
  int normalize;      /* norm_topk_prob */
  float scale;        /* routed_scaling_factor */
  const uint16_t* router;      /* [E,H] bf16 */
  const uint16_t* gate;        /* [E,I,H] bf16 */
  const uint16_t* up;          /* [E,I,H] bf16 */
  const uint16_t* down;        /* [E,H,I] bf16 */
  const uint16_t* shared_gate; /* [S,H] bf16 */
  const uint16_t* shared_up;   /* [S,H] bf16 */
  const uint16_t* shared_down; /* [H,S] bf16 */
  /* Optional INT8 overlay (src/cpu/quantized.rs:239-369): all or none. */
  int quant_mode;               /* ORC_QUANT_* */
  const int8_t* q_gate;         /* [E,I,H] */
  const float* q_gate_s;        /* [E,I,H/32] */
  const int8_t* q_up;
  const float* q_up_s;
  const int8_t* q_down;         /* [E,H,I] */
  const float* q_down_s;        /* [E,H,I/32] */
  const int8_t* q_shared_gate;  /* [S,H] */
  const float* q_shared_gate_s;
  const int8_t* q_shared_up;
  const float* q_shared_up_s;
  const int8_t* q_shared_down;  /* [H,S] */
  const float* q_shared_down_s;
} orc_moe_layer;

typedef struct orc_moe_trace {
  float* logits;          /* [T,E] router output */
  int32_t* topk_ids;      /* [T,k] in route() order */
  float* topk_weights;    /* [T,k] */
  int32_t* expert_offsets;/* [E+1] start of each expert's assignment list */
  int32_t* perm_rows;     /* [T*k] token row per assignment, expert-major */
  float* perm_weights;    /* [T*k] routing weight per assignment */
} orc_moe_trace;

/* Decoder::experts (src/decoder/mod.rs:124-220). threads > 1 with T == 1
 * runs the shared and selected experts as concurrent tasks like the reference
 * (:142-196); the arithmetic is identical either way. scratch_limit is the
 * CpuContext budget in bytes (src/cpu/mod.rs:73-78); 0 means unlimited. */
int orc_moe_experts(const orc_moe_layer* layer, const float* x, size_t T, float* y, int threads,
                    size_t scratch_limit, orc_moe_trace* trace);
/* Decoder::experts with `threads` workers for what the reference runs on its
 * pool (decode tasks at T == 1, row-parallel GEMV rows above 128 K weight
 * elements) and, when row_threads > 1, the rows of every multi-row scalar
 * GEMM split over row_threads threads (not a reference feature; bit-identical
 * results). Used only to time CPU baselines. */
int orc_moe_experts_threads(const orc_moe_layer* layer, const float* x, size_t T, float* y,
                            int threads, int row_threads);

/* Post-attention half of Decoder::layer (src/decoder/mod.rs:351-363):
 * y = x + experts(rms_norm(x, norm_weight, eps)). */
int orc_moe_block(const orc_moe_layer* layer, const float* norm_weight, float eps, const float* x,
                  size_t T, float* y, int threads);
/* The same block with the rows of every multi-row scalar GEMM split over
 * `row_threads` threads: bit-identical to orc_moe_block, and not what the
 * reference does (its prefill GEMM is serial off macOS, src/cpu/ops.rs:
 * 36-47). Used only to time a stronger CPU baseline. */
int orc_moe_block_rows(const orc_moe_layer* layer, const float* norm_weight, float eps,
                       const float* x, size_t T, float* y, int row_threads);

#ifdef __cplusplus
}
#endif
#endif
