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
