// Wave-level softmax top-k for one token (lane = expert), shared by the
// router kernels and the one-token engine.
#pragma once

#include "common.hpp"

namespace uocr {

struct WaveRoute {
  int id;      // lanes j < K: the j-th selected expert
  float w;     // its routing weight
  bool ok;     // false: non-finite logits (ids are 0..K-1, weights 0)
};

// Softmax as ops::softmax (src/cpu/ops.rs:139-187): reject NaN and +inf,
// subtract the maximum, exp, sum, divide. Then k rounds of wave arg-max on
// the key (probability desc, id asc) of moe::route (src/decoder/moe.rs:19),
// the optional renormalisation sum(top-k, selection order) + 1e-20
// (:21-25) and the scale (:26-28). v holds lane's logit (lanes >= n unused).
__device__ inline WaveRoute route_wave(float v, int n, int K, int normalize, float scale) {
  const int lane = threadIdx.x & 63;
  if (lane >= n) v = -INFINITY;
  const bool bad = lane < n && (isnan(v) || v == INFINITY);
  const float m = wave_max(v);
  WaveRoute r;
  if (__any(bad) || !isfinite(m)) {
    // Distinct ids keep any dispatch built from them a permutation.
    r.id = lane < K ? lane : -1;
    r.w = 0.0f;
    r.ok = false;
    return r;
  }
  const float e = lane < n ? expf(v - m) : 0.0f;
  const float sum = wave_sum(e);
  const float p = e / sum;
  unsigned long long key =
      lane < n ? ((unsigned long long)__float_as_uint(p) << 32) | (0xffffffffu - (uint32_t)lane)
               : 0ull;
  int my_id = -1;
  float my_p = 0.0f;
  float den = -0.0f;
  for (int j = 0; j < K; j++) {
    const unsigned long long best = wave_max_u64(key);
    const int id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
    const float pj = __uint_as_float((uint32_t)(best >> 32));
    if (lane == id) key = 0ull;
    if (lane == j) {
      my_id = id;
      my_p = pj;
    }
    den += pj;
  }
  den = normalize ? den + 1e-20f : 1.0f;
  r.id = my_id;
  r.w = lane < K ? my_p / den * scale : 0.0f;
  r.ok = true;
  return r;
}

}  // namespace uocr

namespace uocr {

struct WaveSel {
  bool ok;                   // false: non-finite logits (then ids 0..K-1, weights 0)
  int rank;                  // selected lanes: position in (probability desc, id asc)
  float p;                   // this lane's probability
  float den;                 // sum of the selected probabilities in selection order
  unsigned long long mask;   // bit e set: expert e selected
};

// Routing of one token by one wave on its own (lane = expert; no LDS, no
// workgroup barrier). The maximum and the softmax sum are 16-lane DPP
// reductions combined over the 4 rows; the probabilities are e / sum as
// ops::softmax computes them, only the order of the 64-term sum differing
// from the reference's sequential one. The selection is K rounds of a wave
// arg-max: the key is the probability's bit pattern plus one (a
// non-negative float orders as its bits; 0 marks lanes out of the race),
// ties go to the lowest lane, i.e. (probability desc, id asc) as
// moe::route sorts (src/decoder/moe.rs:19). Each round's probability is
// added to den in selection order, the renormalisation sum of :21-25.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror
  return v;
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_move_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, dpp_move_u32<0xB1>(v));
  v = max(v, dpp_move_u32<0x4E>(v));
  v = max(v, dpp_move_u32<0x141>(v));
  v = max(v, dpp_move_u32<0x140>(v));
  return v;
}
__device__ inline WaveSel route_wave_sel(float v, int n, int K) {
  const int lane = threadIdx.x & 63;
  const bool live = lane < n;
  const bool bad = __ballot(live && (isnan(v) || v == INFINITY)) != 0ull;
  // Value of lane l (a scalar read).
  auto at = [](float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
  const float vr = row16_max(live ? v : -INFINITY);
  const float m = fmaxf(fmaxf(at(vr, 0), at(vr, 16)), fmaxf(at(vr, 32), at(vr, 48)));
  WaveSel r;
  if (bad || !isfinite(m)) {
    // Distinct ids 0..K-1 with weight 0 keep any dispatch a permutation.
    r.ok = false;
    r.rank = lane;
    r.p = 0.0f;
    r.den = 1.0f;
    r.mask = K >= 64 ? ~0ull : ((1ull << K) - 1ull);
    return r;
  }
  const float ex = live ? expf(v - m) : 0.0f;
  const float sr = row16_sum(ex);
  const float sum = (at(sr, 0) + at(sr, 16)) + (at(sr, 32) + at(sr, 48));
  const float p = ex / sum;
  uint32_t cand = live ? __float_as_uint(p) + 1u : 0u;
  int rank = 64;
  float den = -0.0f;
  for (int j = 0; j < K; j++) {
    const uint32_t cr = row16_max_u32(cand);
    const uint32_t top = max(max((uint32_t)__builtin_amdgcn_readlane((int)cr, 0),
                                 (uint32_t)__builtin_amdgcn_readlane((int)cr, 16)),
                             max((uint32_t)__builtin_amdgcn_readlane((int)cr, 32),
                                 (uint32_t)__builtin_amdgcn_readlane((int)cr, 48)));
    if (top == 0u) break;  // fewer than K experts
    const int id = __ffsll((long long)__ballot(cand == top)) - 1;
    if (lane == id) {
      rank = j;
      cand = 0u;
    }
    den += __uint_as_float(top - 1u);
  }
  r.ok = true;
  r.rank = rank;
  r.p = p;
  r.den = den;
  r.mask = __ballot(rank < K);
  return r;
}

// Routing weight of a selected lane: the renormalisation adds 1e-20 to
// the selection-order sum (src/decoder/moe.rs:21-25), then the scale
// (:26-28).
__device__ __forceinline__ float route_weight(const WaveSel& r, int normalize, float scale) {
  if (!r.ok) return 0.0f;
  const float den = normalize ? r.den + 1e-20f : 1.0f;
  return r.p / den * scale;
}

// Expert of ascending slot s (the s-th set bit of the selection mask).
__device__ __forceinline__ int slot_expert(unsigned long long mask, int s) {
  for (int i = 0; i < s; i++) mask &= mask - 1;
  return __ffsll((long long)mask) - 1;
}

}  // namespace uocr
