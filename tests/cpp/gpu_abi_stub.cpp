// The device half of the C ABI (the functions the HIP library implements in
// csrc/api.cpp) as stubs that report Unsupported. Linked with the host
// sources (csrc/host/*.cpp) into a CPU-only library so that the loaders,
// the JSON parser, SHA-256 and the C++ surface can run under AddressSanitizer
// and UndefinedBehaviorSanitizer. Test infrastructure only.
#include <string>

#include "uocr_moe.h"

namespace {
thread_local std::string g_error;
int unsupported() {
  g_error = "CPU-only build: no GPU entry points";
  return UOCR_ERR_UNSUPPORTED;
}
}  // namespace

namespace uocr::host {
int set_last_error(int status, const char* message) {
  g_error = message;
  return status;
}
}  // namespace uocr::host

extern "C" {

int uocr_gpu_ctx_create(int, size_t, uocr_gpu_ctx** out) {
  if (out) *out = nullptr;
  return unsupported();
}
void uocr_gpu_ctx_destroy(uocr_gpu_ctx*) {}
void* uocr_gpu_ctx_stream(uocr_gpu_ctx*) { return nullptr; }
int uocr_gpu_ctx_synchronize(uocr_gpu_ctx*) { return unsupported(); }
int uocr_gpu_ctx_set_timing(uocr_gpu_ctx*, uint32_t) { return unsupported(); }
int uocr_gpu_ctx_set_wait_limit(uocr_gpu_ctx*, int) { return unsupported(); }
int uocr_gpu_ctx_timings(uocr_gpu_ctx*, uocr_phase_time*, size_t, size_t*) {
  return unsupported();
}
const char* uocr_last_error(const uocr_gpu_ctx*) { return g_error.c_str(); }
size_t uocr_moe_scratch_bytes(const uocr_moe_config*, size_t) { return 0; }
size_t uocr_moe_max_tokens(const uocr_moe_config*) { return 0; }
int uocr_moe_layer_create(uocr_gpu_ctx*, const uocr_moe_config*, const uocr_moe_bf16_weights*,
                          uocr_memory, uocr_moe_layer** out) {
  if (out) *out = nullptr;
  return unsupported();
}
int uocr_moe_layer_attach_int8(uocr_gpu_ctx*, uocr_moe_layer*, const uocr_moe_int8_weights*,
                               uocr_memory, uocr_quant_mode) {
  return unsupported();
}
const char* uocr_moe_layer_precision(const uocr_moe_layer*) { return ""; }
size_t uocr_moe_layer_device_bytes(const uocr_moe_layer*) { return 0; }
void uocr_moe_layer_destroy(uocr_moe_layer*) {}
int uocr_moe_forward_async(uocr_gpu_ctx*, const uocr_moe_layer*, const float*, size_t, float*,
                           uint32_t, const uocr_moe_trace*) {
  return unsupported();
}
int uocr_moe_forward(uocr_gpu_ctx*, const uocr_moe_layer*, const float*, size_t, float*, uint32_t,
                     const uocr_moe_trace*) {
  return unsupported();
}
int uocr_moe_forward_static(const uocr_moe_layer*, const float*, size_t, float*, uint32_t,
                            int32_t*, void*) {
  return unsupported();
}
int uocr_moe_block_forward_async(uocr_gpu_ctx*, const uocr_moe_layer* const*, size_t,
                                 const float*, size_t, float*, uint32_t) {
  return unsupported();
}
int uocr_moe_block_forward(uocr_gpu_ctx*, const uocr_moe_layer* const*, size_t, const float*,
                           size_t, float*, uint32_t) {
  return unsupported();
}
int uocr_route(uocr_gpu_ctx*, const float*, size_t, size_t, size_t, int, float, int32_t*,
               float*) {
  return unsupported();
}
int uocr_linear_bf16(uocr_gpu_ctx*, const float*, size_t, size_t, const uint16_t*, size_t,
                     float*) {
  return unsupported();
}
int uocr_int8_linear(uocr_gpu_ctx*, const int8_t*, const float*, size_t, size_t, const float*,
                     size_t, float*) {
  return unsupported();
}
int uocr_int8_linear_dynamic(uocr_gpu_ctx*, const int8_t*, const float*, size_t, size_t,
                             const float*, float*, int32_t*) {
  return unsupported();
}
int uocr_rms_norm(uocr_gpu_ctx*, const float*, size_t, size_t, const float*, float, float*) {
  return unsupported();
}
int uocr_lm_head_create(uocr_gpu_ctx*, const uocr_lm_head_weights*, uocr_memory,
                        uocr_lm_head** out) {
  if (out) *out = nullptr;
  return unsupported();
}
int uocr_lm_head_logits_async(uocr_gpu_ctx*, const uocr_lm_head*, const float*, size_t, float*) {
  return unsupported();
}
int uocr_lm_head_logits(uocr_gpu_ctx*, const uocr_lm_head*, const float*, size_t, float*) {
  return unsupported();
}
const char* uocr_lm_head_precision(const uocr_lm_head*) { return ""; }
size_t uocr_lm_head_device_bytes(const uocr_lm_head*) { return 0; }
void uocr_lm_head_destroy(uocr_lm_head*) {}

}  // extern "C"
