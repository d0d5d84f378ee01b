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

// LDS staging for route_wave_lds (one token per wave).
struct RouteSmem {
  __attribute__((aligned(16))) float v[64];
  __attribute__((aligned(16))) unsigned long long key[64];
  float selp[64];
};

struct LdsRoute {
  bool ok;                   // false: non-finite logits (then ids 0..K-1, weights 0)
  int rank;                  // this lane's position in (probability desc, id asc)
  float p;                   // this lane's probability
  unsigned long long mask;   // bit e set: expert e selected
};

// Routing of one token by one wave on its own (no workgroup barrier; lane
// = expert), with as few instructions as the math allows: the maximum and
// the softmax sum are 16-lane DPP reductions combined over the 4 rows, each
// lane's rank is the number of larger (probability, -id) keys, read back
// from the wave's own LDS keys (a wave's LDS operations complete in order;
// the wave barriers keep the compiler from moving reads above writes). The
// probabilities are e / sum as ops::softmax computes them; only the order
// of the 64-term sum differs from the reference's sequential one. Also
// fills sm.selp with the selected probabilities in rank order for
// route_wave_weight.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror
  return v;
}
__device__ inline LdsRoute route_wave_lds(float v, int n, int K, RouteSmem& sm) {
  const int lane = threadIdx.x & 63;
  const bool live = lane < n;
  const bool bad = __ballot(live && (isnan(v) || v == INFINITY)) != 0ull;
  // Value of lane l (a scalar read).
  auto at = [](float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
  const float vr = row16_max(live ? v : -INFINITY);
  const float m = fmaxf(fmaxf(at(vr, 0), at(vr, 16)), fmaxf(at(vr, 32), at(vr, 48)));
  LdsRoute r;
  if (bad || !isfinite(m)) {
    // Distinct ids 0..K-1 with weight 0 keep any dispatch a permutation.
    r.ok = false;
    r.rank = lane;
    r.p = 0.0f;
    r.mask = K >= 64 ? ~0ull : ((1ull << K) - 1ull);
    return r;
  }
  const float ex = live ? expf(v - m) : 0.0f;
  const float sr = row16_sum(ex);
  const float sum = (at(sr, 0) + at(sr, 16)) + (at(sr, 32) + at(sr, 48));
  const float p = ex / sum;
  const unsigned long long key =
      live ? ((unsigned long long)__float_as_uint(p) << 32) | (0xffffffffu - (uint32_t)lane) : 0ull;
  sm.key[lane] = key;
  __builtin_amdgcn_wave_barrier();
  int rank = 0;
#pragma unroll
  for (int e = 0; e < 64; e += 2) {
    const ulonglong2 u = *reinterpret_cast<const ulonglong2*>(&sm.key[e]);
    rank += (u.x > key ? 1 : 0) + (u.y > key ? 1 : 0);
  }
  r.ok = true;
  r.rank = rank;
  r.p = p;
  r.mask = __ballot(live && rank < K);
  if (live && rank < K) sm.selp[rank] = p;
  __builtin_amdgcn_wave_barrier();
  return r;
}

// Routing weights of the selected lanes (route_wave_lds ranks < K): the
// renormalisation sums the top-k probabilities in selection order
// (src/decoder/moe.rs:21-25), then scales (:26-28).
__device__ inline float route_wave_weight(const LdsRoute& r, int K, int normalize, float scale,
                                          const RouteSmem& sm) {
  if (!r.ok) return 0.0f;
  float den = -0.0f;
  for (int j = 0; j < K; j++) den += sm.selp[j];
  den = normalize ? den + 1e-20f : 1.0f;
  return r.p / den * scale;
}

// Expert of ascending slot s (the s-th set bit of the selection mask).
__device__ __forceinline__ int slot_expert(unsigned long long mask, int s) {
  for (int i = 0; i < s; i++) mask &= mask - 1;
  return __ffsll((long long)mask) - 1;
}

}  // namespace uocr
