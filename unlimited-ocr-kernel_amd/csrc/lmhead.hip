// Vocabulary projection of the last hidden row: Decoder::logits
// (src/decoder/mod.rs:367-379) = RMSNorm with model.norm.weight, then
// Decoder::projection with lm_head.weight (:99-112): BF16 weights widened,
// the INT8 overlay weight-only, or W8A8 when the mode is DynamicActivations
// (the projected row is always a single row there).
//
// One launch: every workgroup normalises the row itself (a few KB; the
// workgroup form of the norm's fixed-order reduction, which the standalone
// norm takes above 1280 wide — up to 1280 it reduces per wave, so the two
// agree to rounding there) into LDS, then its
// four waves stream their 32 rows each of the [V, H] matrix, eight rows per
// pass (16 lanes per row), with the next pass's loads issued before the
// current pass is dotted. The bound is HBM: V * H * (2 | 1 + 4/32) bytes.
#include "common.hpp"
#include "moe_kernels.hpp"
#include "rowdot.hpp"
#include "rownorm.hpp"

namespace uocr {

constexpr int kLmPasses = 4;                              // passes per wave
constexpr int kLmRowsPerWave = 8 * kLmPasses;             // rows per wave
constexpr int kLmRowsPerWg = 4 * kLmRowsPerWave;          // rows per workgroup

template <int KIND, int KMAX>
__global__ __launch_bounds__(kRowThreads) void lm_head_kernel(const float* __restrict__ hidden,
                                                              LmHeadView head,
                                                              float* __restrict__ logits,
                                                              int* err) {
  __shared__ __attribute__((aligned(16))) float xl[KMAX];
  __shared__ __attribute__((aligned(16))) int8_t xq[KIND == kW8A8 ? KMAX : 16];
  __shared__ float xs[KIND == kW8A8 ? KMAX / kQBlock : 1];
  const int H = head.H;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // ---- this wave's rows [r0, r0 + kLmRowsPerWave), eight per pass: the
  // 16-lane group g takes rows 2g and 2g + 1 of the pass. The resources
  // start at r0, so offsets stay small whatever the matrix size. The first
  // pass's loads are issued before the norm, which does not feed them
  // (not for INT8 weight-only: its registers then exceed one SIMD's share
  // for two waves, measured 40 -> 47 us).
  const int r0 = blockIdx.x * kLmRowsPerWg + wave * kLmRowsPerWave;
  const int nrows = min(kLmRowsPerWave, head.V - r0);
  const int nblk = H / kQBlock;
  const void* wbase = KIND == kBF16
                          ? static_cast<const void*>(head.w + (size_t)r0 * H)
                          : static_cast<const void*>(head.q + (size_t)r0 * H);
  const float* sbase = KIND == kBF16 ? nullptr : head.s + (size_t)r0 * nblk;
  const int grp = lane >> 4;
  const int j = lane & 15;
  using RP = RowPair<KIND == kBF16 ? kBF16 : kInt8, KMAX>;
  constexpr bool kDouble = RP::kC <= 10;  // two passes in flight when registers allow
  RP P[kDouble ? 2 : 1];
  constexpr bool kEarly = KIND != kInt8;
  if (kEarly && r0 < head.V) issue_rows(P[0], wbase, sbase, nrows, H, 2 * grp, 2 * grp + 1);

  // ---- RMSNorm of the row into LDS.
  float4 row[kRowChunks];
#pragma unroll
  for (int it = 0; it < kRowChunks; it++) {
    const int i = (tid + kRowThreads * it) * 4;
    if (i >= H) break;
    row[it] = *reinterpret_cast<const float4*>(hidden + i);
  }
  norm_row(row, H, head.norm_w, head.eps, xl, nullptr, nullptr, blockIdx.x == 0 ? err : nullptr);
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    quantize_lds_waves(xl, H, xq, xs, wave, kRowThreads / 64, lane, blockIdx.x == 0 ? err : nullptr);
    __syncthreads();
  }
  if (r0 >= head.V) return;  // no barrier follows
  if (!kEarly) issue_rows(P[0], wbase, sbase, nrows, H, 2 * grp, 2 * grp + 1);

#pragma unroll
  for (int pass = 0; pass < kLmPasses; pass++) {
    RP& cur = P[kDouble ? (pass & 1) : 0];
    if constexpr (kDouble) {
      if (pass + 1 < kLmPasses)
        issue_rows(P[(pass + 1) & 1], wbase, sbase, nrows, H, 8 * (pass + 1) + 2 * grp,
                   8 * (pass + 1) + 2 * grp + 1);
    }
    float a, b;
    dot_rows_as<KIND>(cur, H, xl, xq, xs, a, b);
    if constexpr (!kDouble) {
      if (pass + 1 < kLmPasses)
        issue_rows(P[0], wbase, sbase, nrows, H, 8 * (pass + 1) + 2 * grp,
                   8 * (pass + 1) + 2 * grp + 1);
    }
    const int ra = 8 * pass + 2 * grp;
    if (j == 0) {
      if (ra < nrows) logits[r0 + ra] = a;
      if (ra + 1 < nrows) logits[r0 + ra + 1] = b;
    }
  }
}

bool lm_head_fast(int H) { return H % 64 == 0 && H <= 2048; }

void launch_lm_head(const float* hidden, const LmHeadView& head, float* logits, int* err,
                    hipStream_t s) {
  const dim3 grid((unsigned)((head.V + kLmRowsPerWg - 1) / kLmRowsPerWg)), block(kRowThreads);
  const bool narrow = head.H <= 1280;
#define UOCR_LM(KIND)                                                                \
  do {                                                                               \
    if (narrow)                                                                      \
      lm_head_kernel<KIND, 1280><<<grid, block, 0, s>>>(hidden, head, logits, err);  \
    else                                                                             \
      lm_head_kernel<KIND, 2048><<<grid, block, 0, s>>>(hidden, head, logits, err);  \
  } while (0)
  if (head.kind == kBF16)
    UOCR_LM(kBF16);
  else if (head.kind == kInt8)
    UOCR_LM(kInt8);
  else
    UOCR_LM(kW8A8);
#undef UOCR_LM
}

}  // namespace uocr
