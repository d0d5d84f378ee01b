/*
 * CPU oracle for the Unlimited-OCR MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the reported CPU baseline.
 * Nothing in the product library links, loads or calls this code.
 *
 * This is a restatement of the reference's x86 scalar branches. Sums run in
 * the reference's sequential order starting from -0.0 (Rust's float
 * `iter::Sum`), every multiply and add is rounded separately (the file is
 * built with -ffp-contract=off and without fast-math), and exponentials use
 * glibc expf, which is what Rust's f32::exp resolves to on x86-64 Linux.
 * Threading mirrors the reference's rayon use and never changes a value.
 */
#include "uocr_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define BLOCK 32

typedef struct {
  int threads;
  size_t scratch; /* bytes; 0 = unlimited */
  /* Not a reference semantic: > 1 splits the rows of the multi-row scalar
   * GEMM over that many threads (each row's dot keeps its order, so the
   * result is bit-identical). Only the CPU-baseline timing sets it. */
  int row_threads;
} orc_ctx;

/* src/cpu/mod.rs:73-78: elements * 4 must fit the scratch limit. */
static int check_elements(const orc_ctx* cpu, size_t count) {
  if (cpu->scratch == 0) return ORC_OK;
  if (count > SIZE_MAX / 4 || count * 4 > cpu->scratch) return ORC_RESOURCE;
  return ORC_OK;
}

float orc_bf16_to_f32(uint16_t bits) {
  uint32_t u = (uint32_t)bits << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float value) {
  uint32_t u;
  memcpy(&u, &value, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t round_bit = 0x00008000u;
  if ((u & round_bit) != 0 && (u & (3u * round_bit - 1u)) != 0) return (uint16_t)((u >> 16) + 1u);
  return (uint16_t)(u >> 16);
}

/* ---------------------------------------------------------------- softmax */

/* src/cpu/ops.rs:139-187, Backend::Scalar on x86: reject empty rows, NaN and
 * +inf; max by fold(-inf, max); subtract; expf; sequential sum; divide. */
int orc_softmax(float* v, size_t n) {
  if (n == 0) return ORC_NUMERICAL;
  for (size_t i = 0; i < n; i++)
    if (isnan(v[i]) || v[i] == INFINITY) return ORC_NUMERICAL;
  float maximum = -INFINITY;
  for (size_t i = 0; i < n; i++) maximum = fmaxf(maximum, v[i]);
  if (!isfinite(maximum)) return ORC_NUMERICAL;
  for (size_t i = 0; i < n; i++) v[i] -= maximum;
  for (size_t i = 0; i < n; i++) v[i] = expf(v[i]);
  float sum = -0.0f;
  for (size_t i = 0; i < n; i++) sum += v[i];
  for (size_t i = 0; i < n; i++) v[i] /= sum;
  return ORC_OK;
}

/* Rust f32::total_cmp key: flip the magnitude bits of negatives. */
static int32_t total_key(float f) {
  int32_t b;
  memcpy(&b, &f, 4);
  b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
  return b;
}

/* src/decoder/moe.rs:7-30. */
int orc_route(const float* logits, size_t n, size_t count, int normalize, float scale,
              int32_t* ids, float* weights) {
  if (count == 0 || count > n || !isfinite(scale) || scale <= 0.0f) return ORC_SHAPE;
  float* p = (float*)malloc(n * sizeof(float));
  size_t* order = (size_t*)malloc(n * sizeof(size_t));
  if (!p || !order) {
    free(p);
    free(order);
    return ORC_RESOURCE;
  }
  memcpy(p, logits, n * sizeof(float));
  int st = orc_softmax(p, n);
  if (st != ORC_OK) {
    free(p);
    free(order);
    return st;
  }
  /* Sort by (probability descending under total_cmp, id ascending). The key
   * pairs are unique, so any correct sort yields the reference's order;
   * insertion sort keeps this dependency-free. */
  for (size_t i = 0; i < n; i++) {
    size_t j = i;
    int32_t ki = total_key(p[i]);
    while (j > 0) {
      size_t prev = order[j - 1];
      int32_t kp = total_key(p[prev]);
      if (kp > ki || (kp == ki && prev < i)) break;
      order[j] = prev;
      j--;
    }
    order[j] = i;
  }
  float denominator = 1.0f;
  if (normalize) {
    float sum = -0.0f;
    for (size_t j = 0; j < count; j++) sum += p[order[j]];
    denominator = sum + 1e-20f;
  }
  for (size_t j = 0; j < count; j++) {
    ids[j] = (int32_t)order[j];
    weights[j] = p[order[j]] / denominator * scale;
  }
  free(p);
  free(order);
  return ORC_OK;
}

/* ------------------------------------------------------------ dense linear */

static int linear_ctx(const orc_ctx* cpu, const float* x, size_t m, size_t k, const float* w,
                      size_t n, const float* bias, float* y) {
  if (k == 0 || n == 0) return ORC_SHAPE;
  if (m != 0 && n > SIZE_MAX / m) return ORC_SHAPE;
  int st = check_elements(cpu, m * n);
  if (st) return st;
  /* src/cpu/ops.rs:39-47: single-threaded scalar triple loop off macOS. */
#pragma omp parallel for num_threads(cpu->row_threads) schedule(static) if (cpu->row_threads > 1)
  for (size_t i = 0; i < m; i++) {
    const float* xr = x + i * k;
    for (size_t j = 0; j < n; j++) {
      const float* wr = w + j * k;
      float acc = -0.0f;
      for (size_t t = 0; t < k; t++) acc += xr[t] * wr[t];
      y[i * n + j] = acc;
    }
  }
  if (bias) {
    for (size_t i = 0; i < m; i++)
      for (size_t j = 0; j < n; j++) y[i * n + j] += bias[j];
  }
  return ORC_OK;
}

int orc_linear(const float* x, size_t m, size_t k, const float* w, size_t n, const float* bias,
               float* y) {
  orc_ctx cpu = {1, 0, 0};
  return linear_ctx(&cpu, x, m, k, w, n, bias, y);
}

/* src/cpu/ops.rs:62-133. */
static int linear_weight_ctx(const orc_ctx* cpu, const float* x, size_t m, size_t k,
                             const uint16_t* w, size_t n, const float* bias, float* y) {
  if (k == 0 || n == 0) return ORC_SHAPE;
  if (m == 1) {
    int st = check_elements(cpu, n);
    if (st) return st;
    /* :87-103 scalar GEMV row, then `+ bias.map_or(0., ..)`; :104-115 rows
     * run in parallel above 128 K weight elements. */
    int parallel = cpu->threads > 1 && n * k > 128 * 1024;
#pragma omp parallel for num_threads(cpu->threads) schedule(static) if (parallel)
    for (size_t row = 0; row < n; row++) {
      const uint16_t* wr = w + row * k;
      float acc = -0.0f;
      for (size_t t = 0; t < k; t++) acc += orc_bf16_to_f32(wr[t]) * x[t];
      y[row] = acc + (bias ? bias[row] : 0.0f);
    }
    return ORC_OK;
  }
  /* :119-132: widen the whole matrix to f32, then the scalar GEMM. */
  if (m != 0 && n > SIZE_MAX / m) return ORC_RESOURCE;
  int st = check_elements(cpu, n * k + m * n);
  if (st) return st;
  float* wide = (float*)malloc(n * k * sizeof(float));
  if (!wide) return ORC_RESOURCE;
  for (size_t i = 0; i < n * k; i++) wide[i] = orc_bf16_to_f32(w[i]);
  st = linear_ctx(cpu, x, m, k, wide, n, bias, y);
  free(wide);
  return st;
}

int orc_linear_weight_bf16(const float* x, size_t m, size_t k, const uint16_t* w, size_t n,
                           const float* bias, float* y, int threads) {
  orc_ctx cpu = {threads > 0 ? threads : 1, 0, 0};
  return linear_weight_ctx(&cpu, x, m, k, w, n, bias, y);
}

/* src/cpu/ops.rs:225-229: v / (1 + exp(-v)). */
void orc_silu(float* v, size_t n) {
  for (size_t i = 0; i < n; i++) v[i] /= 1.0f + expf(-v[i]);
}

/* src/cpu/ops.rs:362-423 with center = false (rms_norm, :420-422). */
int orc_rms_norm(const float* x, size_t rows, size_t width, const float* weight, float eps,
                 float* out) {
  if (width == 0 || !isfinite(eps) || eps <= 0.0f) return ORC_SHAPE;
  for (size_t i = 0; i < rows * width; i++)
    if (!isfinite(x[i])) return ORC_NUMERICAL;
  for (size_t i = 0; i < width; i++)
    if (!isfinite(weight[i])) return ORC_NUMERICAL;
  const float mean = 0.0f;
  for (size_t r = 0; r < rows; r++) {
    const float* in = x + r * width;
    float* o = out + r * width;
    float variance = -0.0f;
    for (size_t i = 0; i < width; i++) variance += (in[i] - mean) * (in[i] - mean);
    variance = variance / (float)width;
    float scale = 1.0f / sqrtf(variance + eps);
    for (size_t i = 0; i < width; i++) o[i] = (in[i] - mean) * scale * weight[i] + 0.0f;
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------- INT8 */

static size_t blocks_of(size_t cols) { return (cols + BLOCK - 1) / BLOCK; }

/* src/cpu/quantized.rs:18-42. */
int orc_int8_check(size_t rows, size_t cols, size_t n_weights, size_t n_scales,
                   const float* scales) {
  if (rows == 0 || cols == 0) return ORC_SHAPE;
  if (cols > SIZE_MAX / rows || rows * cols != n_weights) return ORC_SHAPE;
  if (rows * blocks_of(cols) != n_scales) return ORC_SHAPE;
  for (size_t i = 0; i < n_scales; i++)
    if (!isfinite(scales[i]) || scales[i] < 0.0f) return ORC_NUMERICAL;
  return ORC_OK;
}

/* src/cpu/quantized.rs:43-74. */
int orc_int8_quantize(const float* m, size_t rows, size_t cols, int8_t* q, float* s) {
  if (rows == 0 || cols == 0) return ORC_SHAPE;
  for (size_t i = 0; i < rows * cols; i++)
    if (!isfinite(m[i])) return ORC_NUMERICAL;
  size_t blocks = blocks_of(cols);
  for (size_t r = 0; r < rows; r++) {
    for (size_t b = 0; b < blocks; b++) {
      size_t start = b * BLOCK, end = start + BLOCK < cols ? start + BLOCK : cols;
      const float* v = m + r * cols;
      float maximum = 0.0f;
      for (size_t i = start; i < end; i++) maximum = fmaxf(maximum, fabsf(v[i]));
      float scale = maximum / 127.0f;
      if (maximum > 0.0f && scale == 0.0f) return ORC_NUMERICAL;
      s[r * blocks + b] = scale;
      for (size_t i = start; i < end; i++) {
        int8_t out = 0;
        if (scale != 0.0f) {
          float t = rintf(v[i] / scale);
          if (t < -127.0f) t = -127.0f;
          if (t > 127.0f) t = 127.0f;
          out = (int8_t)t;
        }
        q[r * cols + i] = out;
      }
    }
  }
  return ORC_OK;
}

/* src/cpu/quantized.rs:75-95: w as f32 * scale. */
void orc_int8_dequantize(const int8_t* q, const float* s, size_t rows, size_t cols, float* out) {
  size_t blocks = blocks_of(cols);
  for (size_t r = 0; r < rows; r++)
    for (size_t i = 0; i < cols; i++)
      out[r * cols + i] = (float)q[r * cols + i] * s[r * blocks + i / BLOCK];
}

/* src/cpu/quantized.rs:99-150. */
static int int8_linear_ctx(const orc_ctx* cpu, const int8_t* q, const float* s, size_t rows,
                           size_t cols, const float* x, size_t batch, float* y) {
  if (batch != 0 && rows > SIZE_MAX / batch) return ORC_RESOURCE;
  size_t count = batch * rows;
  int st = check_elements(cpu, count);
  if (st) return st;
  if (batch != 1) {
    /* :109-117: dequantize, then the scalar FP32 GEMM. */
    st = check_elements(cpu, rows * cols + count);
    if (st) return st;
    float* deq = (float*)malloc(rows * cols * sizeof(float));
    if (!deq) return ORC_RESOURCE;
    orc_int8_dequantize(q, s, rows, cols, deq);
    st = linear_ctx(cpu, x, batch, cols, deq, rows, NULL, y);
    free(deq);
    return st;
  }
  size_t blocks = blocks_of(cols);
  int parallel = cpu->threads > 1 && rows * cols > 128 * 1024;
  /* :119-131: Σ (w as f32 * scale) * x, sequential over all columns. */
#pragma omp parallel for num_threads(cpu->threads) schedule(static) if (parallel)
  for (size_t row = 0; row < rows; row++) {
    const int8_t* w = q + row * cols;
    const float* sc = s + row * blocks;
    float acc = -0.0f;
    for (size_t i = 0; i < cols; i++) acc += (float)w[i] * sc[i / BLOCK] * x[i];
    y[row] = acc;
  }
  return ORC_OK;
}

int orc_int8_linear(const int8_t* q, const float* s, size_t rows, size_t cols, const float* x,
                    size_t batch, float* y, int threads) {
  orc_ctx cpu = {threads > 0 ? threads : 1, 0, 0};
  return int8_linear_ctx(&cpu, q, s, rows, cols, x, batch, y);
}

/* src/cpu/quantized.rs:155-236. */
static int int8_dynamic_ctx(const orc_ctx* cpu, const int8_t* q, const float* s, size_t rows,
                            size_t cols, const float* x, float* y, int32_t* block_sums) {
  size_t blocks = blocks_of(cols);
  int st = check_elements(cpu, cols * 2 + rows + blocks);
  if (st) return st;
  int8_t* xq = (int8_t*)malloc(cols);
  float* xs = (float*)malloc(blocks * sizeof(float));
  if (!xq || !xs) {
    free(xq);
    free(xs);
    return ORC_RESOURCE;
  }
  st = orc_int8_quantize(x, 1, cols, xq, xs);
  if (st) {
    free(xq);
    free(xs);
    return st;
  }
  int parallel = cpu->threads > 1 && rows * cols > 128 * 1024;
  /* :190-198: per block an exact i32 sum, then (sum as f32 * ws) * xs,
   * accumulated over blocks in order. */
#pragma omp parallel for num_threads(cpu->threads) schedule(static) if (parallel)
  for (size_t row = 0; row < rows; row++) {
    const int8_t* w = q + row * cols;
    const float* ws = s + row * blocks;
    float acc = -0.0f;
    for (size_t b = 0; b < blocks; b++) {
      size_t start = b * BLOCK, end = start + BLOCK < cols ? start + BLOCK : cols;
      int32_t sum = 0;
      for (size_t i = start; i < end; i++) sum += (int32_t)w[i] * (int32_t)xq[i];
      if (block_sums) block_sums[row * blocks + b] = sum;
      acc += (float)sum * ws[b] * xs[b];
    }
    y[row] = acc;
  }
  free(xq);
  free(xs);
  return ORC_OK;
}

int orc_int8_linear_dynamic(const int8_t* q, const float* s, size_t rows, size_t cols,
                            const float* x, float* y, int32_t* block_sums, int threads) {
  orc_ctx cpu = {threads > 0 ? threads : 1, 0, 0};
  return int8_dynamic_ctx(&cpu, q, s, rows, cols, x, y, block_sums);
}

/* -------------------------------------------------------------- MoE layer */

typedef struct {
  const uint16_t* bf16;
  const int8_t* q;
  const float* s;
  size_t n, k;
} matrix;

/* Decoder::projection (src/decoder/mod.rs:99-112). */
static int projection(const orc_ctx* cpu, const orc_moe_layer* L, matrix m, const float* x,
                      size_t rows, float* y) {
  if (L->quant_mode != ORC_QUANT_NONE && m.q) {
    if (L->quant_mode == ORC_QUANT_DYNAMIC && rows == 1)
      return int8_dynamic_ctx(cpu, m.q, m.s, m.n, m.k, x, y, NULL);
    return int8_linear_ctx(cpu, m.q, m.s, m.n, m.k, x, rows, y);
  }
  return linear_weight_ctx(cpu, x, rows, m.k, m.bf16, m.n, NULL, y);
}

/* Decoder::feed_forward (src/decoder/mod.rs:114-122). */
static int feed_forward(const orc_ctx* cpu, const orc_moe_layer* L, matrix g, matrix u, matrix d,
                        const float* x, size_t rows, float* y) {
  size_t width = g.n;
  float* gate = (float*)malloc(rows * width * sizeof(float) + 1);
  float* up = (float*)malloc(rows * width * sizeof(float) + 1);
  int st = (!gate || !up) ? ORC_RESOURCE : ORC_OK;
  if (!st) st = projection(cpu, L, g, x, rows, gate);
  if (!st) st = projection(cpu, L, u, x, rows, up);
  if (!st) {
    orc_silu(gate, rows * width);
    for (size_t i = 0; i < rows * width; i++) gate[i] *= up[i];
    st = projection(cpu, L, d, gate, rows, y);
  }
  free(gate);
  free(up);
  return st;
}

static void expert_matrices(const orc_moe_layer* L, size_t e, matrix* g, matrix* u, matrix* d) {
  size_t H = L->hidden, I = L->inter;
  size_t bh = blocks_of(H), bi = blocks_of(I);
  *g = (matrix){L->gate ? L->gate + e * I * H : NULL, L->q_gate ? L->q_gate + e * I * H : NULL,
                L->q_gate_s ? L->q_gate_s + e * I * bh : NULL, I, H};
  *u = (matrix){L->up ? L->up + e * I * H : NULL, L->q_up ? L->q_up + e * I * H : NULL,
                L->q_up_s ? L->q_up_s + e * I * bh : NULL, I, H};
  *d = (matrix){L->down ? L->down + e * H * I : NULL, L->q_down ? L->q_down + e * H * I : NULL,
                L->q_down_s ? L->q_down_s + e * H * bi : NULL, H, I};
}

static void shared_matrices(const orc_moe_layer* L, matrix* g, matrix* u, matrix* d) {
  size_t H = L->hidden, S = L->shared;
  *g = (matrix){L->shared_gate, L->q_shared_gate, L->q_shared_gate_s, S, H};
  *u = (matrix){L->shared_up, L->q_shared_up, L->q_shared_up_s, S, H};
  *d = (matrix){L->shared_down, L->q_shared_down, L->q_shared_down_s, H, S};
}

static int validate_layer(const orc_moe_layer* L) {
  if (!L || L->hidden == 0 || L->inter == 0 || L->shared == 0 || L->n_experts == 0)
    return ORC_SHAPE;
  if (L->top_k == 0 || L->top_k > L->n_experts) return ORC_SHAPE;
  if (!L->router) return ORC_SHAPE;
  if (L->quant_mode != ORC_QUANT_NONE && L->quant_mode != ORC_QUANT_WEIGHTS_ONLY &&
      L->quant_mode != ORC_QUANT_DYNAMIC)
    return ORC_UNSUPPORTED;
  if (L->quant_mode == ORC_QUANT_NONE) {
    if (!L->gate || !L->up || !L->down || !L->shared_gate || !L->shared_up || !L->shared_down)
      return ORC_SHAPE;
  } else {
    /* Model::load_with_quantization: dynamic mode needs an overlay
     * (src/model/mod.rs:87-92). */
    if (!L->q_gate || !L->q_up || !L->q_down || !L->q_shared_gate || !L->q_shared_up ||
        !L->q_shared_down || !L->q_gate_s || !L->q_up_s || !L->q_down_s ||
        !L->q_shared_gate_s || !L->q_shared_up_s || !L->q_shared_down_s)
      return ORC_FORMAT;
  }
  return ORC_OK;
}

static int experts_ctx(const orc_ctx* cpu, const orc_moe_layer* L, const float* x, size_t T,
                       float* y, orc_moe_trace* trace) {
  int st = validate_layer(L);
  if (st) return st;
  size_t H = L->hidden, E = L->n_experts, K = L->top_k;
  matrix router = {L->router, NULL, NULL, E, H};
  float* logits = (float*)malloc(T * E * sizeof(float) + 1);
  int32_t* ids = (int32_t*)malloc(T * K * sizeof(int32_t) + 1);
  float* weights = (float*)malloc(T * K * sizeof(float) + 1);
  int32_t* counts = (int32_t*)calloc(E + 1, sizeof(int32_t));
  int32_t* rows = (int32_t*)malloc(T * K * sizeof(int32_t) + 1);
  float* probs = (float*)malloc(T * K * sizeof(float) + 1);
  float* work = NULL;
  if (!logits || !ids || !weights || !counts || !rows || !probs) {
    st = ORC_RESOURCE;
    goto done;
  }
  /* :126 router logits; the gate matrix is never in the INT8 overlay. */
  st = linear_weight_ctx(cpu, x, T, H, L->router, E, NULL, logits);
  if (st) goto done;
  (void)router;
  /* :127-141 route every row; assignments[e] collects rows in order. */
  for (size_t t = 0; t < T; t++) {
    st = orc_route(logits + t * E, E, K, L->normalize, L->scale, ids + t * K, weights + t * K);
    if (st) goto done;
  }
  for (size_t t = 0; t < T; t++)
    for (size_t j = 0; j < K; j++) counts[ids[t * K + j] + 1]++;
  for (size_t e = 0; e < E; e++) counts[e + 1] += counts[e];
  {
    int32_t* fill = (int32_t*)malloc(E * sizeof(int32_t));
    if (!fill) {
      st = ORC_RESOURCE;
      goto done;
    }
    memcpy(fill, counts, E * sizeof(int32_t));
    for (size_t t = 0; t < T; t++)
      for (size_t j = 0; j < K; j++) {
        int32_t e = ids[t * K + j];
        rows[fill[e]] = (int32_t)t;
        probs[fill[e]] = weights[t * K + j];
        fill[e]++;
      }
    free(fill);
  }
  if (trace) {
    if (trace->logits) memcpy(trace->logits, logits, T * E * sizeof(float));
    if (trace->topk_ids) memcpy(trace->topk_ids, ids, T * K * sizeof(int32_t));
    if (trace->topk_weights) memcpy(trace->topk_weights, weights, T * K * sizeof(float));
    if (trace->expert_offsets) memcpy(trace->expert_offsets, counts, (E + 1) * sizeof(int32_t));
    if (trace->perm_rows) memcpy(trace->perm_rows, rows, T * K * sizeof(int32_t));
    if (trace->perm_weights) memcpy(trace->perm_weights, probs, T * K * sizeof(float));
  }
  matrix sg, su, sd;
  shared_matrices(L, &sg, &su, &sd);

  if (T == 1 && cpu->threads > 1) {
    /* :142-196: shared expert plus each selected expert as a pool task,
     * accumulated in ascending expert order. */
    size_t selected = 0;
    for (size_t e = 0; e < E; e++) selected += counts[e + 1] > counts[e];
    size_t tasks = selected + 1;
    size_t width = L->shared; /* moe_intermediate_size * max(n_shared, 1) */
    size_t need = ((width + H) * 3 + width * H) * tasks;
    if (selected > 0 && check_elements(cpu, need) == ORC_OK) {
      int32_t* task_expert = (int32_t*)malloc(tasks * sizeof(int32_t));
      float* task_p = (float*)malloc(tasks * sizeof(float));
      int* task_status = (int*)calloc(tasks, sizeof(int));
      work = (float*)malloc(tasks * H * sizeof(float));
      if (!task_expert || !task_p || !task_status || !work) {
        free(task_expert);
        free(task_p);
        free(task_status);
        st = ORC_RESOURCE;
        goto done;
      }
      size_t n = 1;
      task_expert[0] = -1;
      for (size_t e = 0; e < E; e++)
        if (counts[e + 1] > counts[e]) {
          task_expert[n] = (int32_t)e;
          task_p[n] = probs[counts[e]];
          n++;
        }
      orc_ctx worker = {1, cpu->scratch ? cpu->scratch / tasks : 0, 0};
#pragma omp parallel for num_threads(cpu->threads) schedule(dynamic, 1)
      for (size_t task = 0; task < tasks; task++) {
        matrix g, u, d;
        if (task == 0) {
          g = sg;
          u = su;
          d = sd;
        } else {
          expert_matrices(L, (size_t)task_expert[task], &g, &u, &d);
        }
        task_status[task] = feed_forward(&worker, L, g, u, d, x, 1, work + task * H);
      }
      for (size_t task = 0; task < tasks && !st; task++) st = task_status[task];
      if (!st) {
        memcpy(y, work, H * sizeof(float));
        for (size_t task = 1; task < tasks; task++)
          for (size_t i = 0; i < H; i++) y[i] += task_p[task] * work[task * H + i];
      }
      free(task_expert);
      free(task_p);
      free(task_status);
      goto done;
    }
  }
  /* :197-219: shared expert over all rows, then every expert in ascending id:
   * gather its rows, run the FFN, y[row] += p * output. */
  st = feed_forward(cpu, L, sg, su, sd, x, T, y);
  if (st) goto done;
  work = (float*)malloc((T * H * 2 + 1) * sizeof(float));
  if (!work) {
    st = ORC_RESOURCE;
    goto done;
  }
  for (size_t e = 0; e < E && !st; e++) {
    size_t n = (size_t)(counts[e + 1] - counts[e]);
    if (n == 0) continue;
    float* input = work;
    float* output = work + T * H;
    for (size_t r = 0; r < n; r++)
      memcpy(input + r * H, x + (size_t)rows[counts[e] + r] * H, H * sizeof(float));
    matrix g, u, d;
    expert_matrices(L, e, &g, &u, &d);
    st = feed_forward(cpu, L, g, u, d, input, n, output);
    if (st) break;
    for (size_t r = 0; r < n; r++) {
      float p = probs[counts[e] + r];
      float* dest = y + (size_t)rows[counts[e] + r] * H;
      for (size_t i = 0; i < H; i++) dest[i] += p * output[r * H + i];
    }
  }
done:
  free(logits);
  free(ids);
  free(weights);
  free(counts);
  free(rows);
  free(probs);
  free(work);
  return st;
}

int orc_moe_experts(const orc_moe_layer* layer, const float* x, size_t T, float* y, int threads,
                    size_t scratch_limit, orc_moe_trace* trace) {
  orc_ctx cpu = {threads > 0 ? threads : 1, scratch_limit, 0};
  return experts_ctx(&cpu, layer, x, T, y, trace);
}

int orc_moe_experts_threads(const orc_moe_layer* layer, const float* x, size_t T, float* y,
                            int threads, int row_threads) {
  orc_ctx cpu = {threads > 0 ? threads : 1, 0, row_threads};
  return experts_ctx(&cpu, layer, x, T, y, NULL);
}

static int moe_block_ctx(const orc_ctx* cpu, const orc_moe_layer* layer,
                         const float* norm_weight, float eps, const float* x, size_t T, float* y) {
  if (!layer) return ORC_SHAPE;
  size_t H = layer->hidden;
  float* normalized = (float*)malloc(T * H * sizeof(float) + 1);
  if (!normalized) return ORC_RESOURCE;
  int st = orc_rms_norm(x, T, H, norm_weight, eps, normalized);
  if (!st) st = experts_ctx(cpu, layer, normalized, T, y, NULL);
  if (!st) {
    /* src/decoder/mod.rs:361-363: residual += mlp. */
    for (size_t i = 0; i < T * H; i++) y[i] = x[i] + y[i];
  }
  free(normalized);
  return st;
}

int orc_moe_block(const orc_moe_layer* layer, const float* norm_weight, float eps, const float* x,
                  size_t T, float* y, int threads) {
  orc_ctx cpu = {threads > 0 ? threads : 1, 0, 0};
  return moe_block_ctx(&cpu, layer, norm_weight, eps, x, T, y);
}

int orc_moe_block_rows(const orc_moe_layer* layer, const float* norm_weight, float eps,
                       const float* x, size_t T, float* y, int row_threads) {
  orc_ctx cpu = {1, 0, row_threads};
  return moe_block_ctx(&cpu, layer, norm_weight, eps, x, T, y);
}
