// The router logits of a one-token launch, handed from its logit
// workgroups to its routed gate/up workgroups: routed workgroup i owns a
// copy of 64 words at word kDecodeCopyWord + 64 i of Scratch::part. A copy
// holds the sentinel 0xffffffff between launches; the logit workgroups
// store their logits into every copy device-coherently (a value with the
// sentinel's bits becomes the quiet NaN 0x7fc00000), the routed workgroup
// polls its copy until no word below E is the sentinel and, once done
// with it, writes the sentinel back. Every word has one writer and one
// reader per launch and no line is polled by two workgroups (hundreds of
// waves polling one line serialise where the XCDs meet).
#pragma once

#include "common.hpp"
#include "moe_kernels.hpp"
#include "rowdot.hpp"

namespace uocr {

constexpr uint32_t kSlotSentinel = 0xffffffffu;
constexpr int kCopyWords = 64;
// The copies follow the split-K engine's partials.
constexpr size_t kDecodeCopyWord = (size_t)(2048 / 32 + 8 * 1024 / 32) * 2048;
static_assert((kDecodeCopyWord + (size_t)8 * 1024 / 32 * kCopyWords) * 4 <= kDecodePartBytes,
              "logit copies fit the part region");

// The bits a slot receives for v: never the sentinel's.
__device__ __forceinline__ uint32_t publish_bits(float v) {
  const uint32_t bits = __float_as_uint(v);
  return bits == kSlotSentinel ? 0x7fc00000u : bits;
}
// Device-coherent 4-byte store of a value that another workgroup reads.
__device__ __forceinline__ void slot_store(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t* logit_copy(float* part, int i) {
  return reinterpret_cast<uint32_t*>(part) + kDecodeCopyWord + (size_t)i * kCopyWords;
}

// Logit workgroup b's 8 logits (rows 8b .. 8b+7, in LDS) into the copies of
// routed workgroups 0 .. n_routed: wave w of nw stores rows 8b + (lane & 7)
// below E into copies 8 w + lane / 8, + 8 nw, ...
__device__ __forceinline__ void publish_logits(float* part, const float* logits8, int b, int E,
                                               int n_routed, int wave, int nw, int lane) {
  const int j = lane & 7, row = 8 * b + j;
  if (row >= E) return;
  const uint32_t v = publish_bits(logits8[j]);
  for (int i = 8 * wave + (lane >> 3); i < n_routed; i += 8 * nw)
    slot_store(logit_copy(part, i) + row, v);
}

// One wave: polls routed workgroup i's copy until no word below E is the
// sentinel, at most `bound` times (then Resource is raised and a word still
// the sentinel reads as 0, so the forward reports Resource rather than a
// NaN). Lane e returns logit e (0 past E).
__device__ __forceinline__ float poll_logits(float* part, int i, int E, int bound, int* err,
                                             int lane) {
  constexpr int kCoherentLoad = 16;  // buffer-load cache policy: sc1 (device coherent)
  const __amdgpu_buffer_rsrc_t cr = make_rsrc(logit_copy(part, i), (uint32_t)E * 4u);
  uint32_t v = 0u;
  for (int it = 0;; it++) {
    v = __builtin_amdgcn_raw_buffer_load_b32(cr, lane < E ? (uint32_t)lane * 4u : kOut, 0,
                                             kCoherentLoad);
    if (__ballot(lane < E && v == kSlotSentinel) == 0ull) break;
    if (it >= bound) {
      if (lane == 0) raise_error(err, 6);  // uocr_status Resource
      break;
    }
    __builtin_amdgcn_s_sleep(2);
    asm volatile("" ::: "memory");  // the next poll reloads
  }
  return lane < E && v != kSlotSentinel ? __uint_as_float(v) : 0.0f;
}

// The copy back to the sentinel (one wave, after its last read).
__device__ __forceinline__ void release_logits(float* part, int i, int E, int lane) {
  if (lane < E) slot_store(logit_copy(part, i) + lane, kSlotSentinel);
}

}  // namespace uocr
