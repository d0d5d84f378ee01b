// Shared device helpers for the gfx950 MoE kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace uocr {

constexpr int kWave = 64;
constexpr int kQBlock = 32;  // INT8 scale block along K (src/cpu/quantized.rs:9)

// Device error codes share the values of uocr_status.
constexpr int kErrNumerical = 7;

__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// Wave-wide reductions over 64 lanes.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    unsigned long long other = __shfl_xor(v, o);
    v = other > v ? other : v;
  }
  return v;
}
// Sum over aligned groups of 16 lanes.
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ void raise_error(int* err, int code) {
  if (err) atomicMax(err, code);
}

// SiLU exactly as the reference writes it: v / (1 + exp(-v)) (src/cpu/ops.rs:225-229).
__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

}  // namespace uocr
