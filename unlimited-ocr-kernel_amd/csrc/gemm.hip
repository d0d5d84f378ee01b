// MFMA grouped GEMM engine (placeholder until the prefill kernels land).
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {}  // namespace uocr
