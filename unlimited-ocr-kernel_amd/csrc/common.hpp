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

// bf16(a) in the low half, bf16(b) in the high half (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

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

// The same sum with DPP lane moves inside each 16-lane row (no LDS
// crossbar): quad swaps, then the half-row and row mirrors; every lane of
// the row ends with the row's sum.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  return v;
}
// Largest value over each 32-lane half of the wave: the row maximum as
// above, then the two rows of a half exchanged by a swizzle (lane ^ 16).
// Every lane of the wave must be active.
__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  // ds_swizzle bit mode: and 0x1f, or 0, xor 0x10.
  return fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f)));
}

__device__ __forceinline__ void raise_error(int* err, int code) {
  if (err) atomicMax(err, code);
}

// SiLU exactly as the reference writes it: v / (1 + exp(-v)) (src/cpu/ops.rs:225-229).
__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

}  // namespace uocr
