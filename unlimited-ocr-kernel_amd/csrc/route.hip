// Router: gate logits (x . W_gate^T) and softmax top-k per token.
//
// Reference: Decoder::experts computes the logits with linear_weight
// (src/decoder/mod.rs:126) and routes each row with moe::route
// (src/decoder/moe.rs:7-30), whose softmax is ops::softmax
// (src/cpu/ops.rs:139-187).
#include "common.hpp"
#include "moe_kernels.hpp"
#include "routing.hpp"

namespace uocr {

// Few tokens: one wave per expert row streams that row once (coalesced
// 256-byte loads of bf16 pairs) and dots it with every token.
template <int TMAX>
__global__ __launch_bounds__(256) void router_rows_kernel(const float* __restrict__ x,
                                                          const uint16_t* __restrict__ w, int T,
                                                          int H, int E,
                                                          float* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  const uint32_t* row = reinterpret_cast<const uint32_t*>(w + (size_t)e * H);
  const int pairs = H / 2;  // H is a multiple of 128
  float acc[TMAX];
#pragma unroll
  for (int t = 0; t < TMAX; t++) acc[t] = 0.0f;
  for (int p = lane; p < pairs; p += 64) {
    uint32_t wp = row[p];
    float w0 = bf16_lo(wp), w1 = bf16_hi(wp);
    // Every token's pair is loaded before any is used (tokens past T read
    // token 0 again and are not used).
    float2 xv[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; t++)
      xv[t] = reinterpret_cast<const float2*>(x + (size_t)(t < T ? t : 0) * H)[p];
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
      if (t < T) {
        acc[t] = fmaf(w0, xv[t].x, acc[t]);
        acc[t] = fmaf(w1, xv[t].y, acc[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TMAX; t++) {
    if (t < T) {
      float s = wave_sum(acc[t]);
      if (lane == 0) logits[(size_t)t * E + e] = s;
    }
  }
}

// Many tokens: lane = expert, a workgroup owns 16 tokens (4 per wave) and
// stages K-chunks of the router (transposed, bf16 pairs) and of the token
// rows in LDS.
constexpr int kRouterKC = 256;  // K elements per chunk
constexpr int kRouterTok = 16;  // tokens per workgroup

__global__ __launch_bounds__(256) void router_tile_kernel(const float* __restrict__ x,
                                                          const uint16_t* __restrict__ w, int T,
                                                          int H, int E,
                                                          float* __restrict__ logits) {
  __shared__ uint32_t wl[(kRouterKC / 2) * 65];  // [k/2][expert], padded
  __shared__ float xl[kRouterTok][kRouterKC];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int t0 = blockIdx.x * kRouterTok;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < H; k0 += kRouterKC) {
    const int kc = min(kRouterKC, H - k0);  // a multiple of 64
    // Router chunk: E rows x KC/2 pairs (zero past kc).
    for (int i = tid; i < 64 * (kRouterKC / 2); i += 256) {
      int e = i / (kRouterKC / 2), p = i % (kRouterKC / 2);
      uint32_t v = 0;
      if (e < E && 2 * p < kc) v = reinterpret_cast<const uint32_t*>(w + (size_t)e * H + k0)[p];
      wl[p * 65 + e] = v;
    }
    for (int i = tid; i < kRouterTok * (kRouterKC / 4); i += 256) {
      int t = i / (kRouterKC / 4), q = i % (kRouterKC / 4);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (t0 + t < T && 4 * q < kc)
        v = reinterpret_cast<const float4*>(x + (size_t)(t0 + t) * H + k0)[q];
      reinterpret_cast<float4*>(&xl[t][0])[q] = v;
    }
    __syncthreads();
#pragma unroll 4
    for (int p = 0; p < kRouterKC / 2; p++) {
      uint32_t wp = wl[p * 65 + lane];
      float w0 = bf16_lo(wp), w1 = bf16_hi(wp);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float2 xv = *reinterpret_cast<const float2*>(&xl[wave * 4 + j][2 * p]);
        acc[j] = fmaf(w0, xv.x, acc[j]);
        acc[j] = fmaf(w1, xv.y, acc[j]);
      }
    }
    __syncthreads();
  }
  if (lane < E) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int t = t0 + wave * 4 + j;
      if (t < T) logits[(size_t)t * E + lane] = acc[j];
    }
  }
}

void launch_router_logits(const float* x, const uint16_t* w, int T, int H, int E, float* logits,
                          hipStream_t s) {
  if (T <= 0) return;
  if (T <= 4) {
    hipLaunchKernelGGL(router_rows_kernel<4>, dim3((E + 3) / 4), dim3(256), 0, s, x, w, T, H, E,
                       logits);
  } else if (T <= 16) {
    hipLaunchKernelGGL(router_rows_kernel<16>, dim3((E + 3) / 4), dim3(256), 0, s, x, w, T, H, E,
                       logits);
  } else {
    hipLaunchKernelGGL(router_tile_kernel, dim3((T + kRouterTok - 1) / kRouterTok), dim3(256), 0,
                       s, x, w, T, H, E, logits);
  }
}

// Routes one token (lane = expert) and writes slots j < K; returns the id
// this lane wrote (-1 for lanes >= K). Non-finite logits raise Numerical.
__device__ int route_token(float v, int n, int K, int normalize, float scale, int* ids,
                           float* weights, int* err) {
  const int lane = threadIdx.x & 63;
  const WaveRoute r = route_wave(v, n, K, normalize, scale);
  if (!r.ok && lane == 0) raise_error(err, kErrNumerical);
  if (lane < K) {
    ids[lane] = r.id;
    weights[lane] = r.w;
  }
  return lane < K ? r.id : -1;
}

// One wave per token.
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ logits, int T, int n,
                                                   int K, int normalize, float scale,
                                                   int* __restrict__ ids,
                                                   float* __restrict__ weights, int* err) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float v = lane < n ? logits[(size_t)t * n + lane] : -INFINITY;
  route_token(v, n, K, normalize, scale, ids + (size_t)t * K, weights + (size_t)t * K, err);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Many tokens: logits on MFMA (v_mfma_f32_16x16x32_bf16), then softmax
// top-k, fused. Each FP32 activation splits exactly into three bf16 terms
// (hi + mid + lo carry its 24 significand bits) and the router weights are
// bf16, so every product is exact and the logits are FP32-accurate sums.
// A workgroup owns 16 tokens and all <= 64 experts; its 4 waves take every
// 4th 32-wide K step and their partial sums are added in wave order
// (deterministic). It also emits the chunk's per-expert assignment counts
// for the dispatch scan.
constexpr int kRouteChunk = 16;
constexpr int kMaxRouteSplit = 8;  // most workgroups per chunk (router_ksplit)

constexpr int kRouteWaves = 8;

// Routes tokens t0 .. t0+15 from their logits v(tl, lane) (two tokens per
// wave): stores logits, ids and weights, and the chunk's per-expert counts.
template <typename LogitOf>
__device__ __forceinline__ void route_chunk(LogitOf logit_of, int chunk, int T, int E, int K,
                                            int normalize, float scale, float* __restrict__ logits,
                                            int* __restrict__ ids, float* __restrict__ weights,
                                            int* __restrict__ chunk_counts, int* cnt, int* err) {
  const int t0 = chunk * kRouteChunk;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  for (int j = 0; j < kRouteChunk / kRouteWaves; j++) {
    const int tl = wave * (kRouteChunk / kRouteWaves) + j;
    const int t = t0 + tl;
    const bool live = t < T;
    const float v = logit_of(tl, lane);
    if (live && lane < E) logits[(size_t)t * E + lane] = v;
    const WaveSel r = route_wave_sel(live ? v : 0.0f, E, K);
    const float wgt = route_weight(r, normalize, scale);
    if (!live) continue;
    if (!r.ok && lane == 0) raise_error(err, kErrNumerical);
    if ((r.mask >> lane) & 1ull) {
      ids[(size_t)t * K + r.rank] = lane;
      weights[(size_t)t * K + r.rank] = wgt;
      atomicAdd(&cnt[lane], 1);
    }
  }
  __syncthreads();
  if (tid < 64) chunk_counts[(size_t)chunk * 64 + tid] = cnt[tid];
}

// KS = K steps (32 wide) per wave. Unsplit (ksplit = 1): workgroup c owns
// tokens 16c.. and wave w takes steps w, w + 8, ...; it reduces, routes and
// counts the chunk. Split (ksplit > 1, few tokens): workgroup c ksplit + p
// takes steps p, p + ksplit, ... (wave w: p + ksplit (w + 8 i)) and writes
// its partial logits [16][64] to part_out[c ksplit + p] with device-coherent
// stores; once they are complete it counts itself in route_counts[16 c], and
// the chunk's last workgroup (the one that sees ksplit - 1) zeroes that word,
// adds the ksplit partials in order (device-coherent loads) and routes the
// chunk. No workgroup waits for another. Steps past H / 32 read as zero. All
// loads of a wave are issued before its MFMAs.
template <int KS>
__global__ __launch_bounds__(64 * kRouteWaves) void router_mfma_kernel(
    const float* __restrict__ x, const uint16_t* __restrict__ w, int T, int H, int E, int K,
    int normalize, float scale, float* __restrict__ logits, int* __restrict__ ids,
    float* __restrict__ weights, int* __restrict__ chunk_counts, uint16_t* __restrict__ x_hi,
    uint16_t* __restrict__ x_lo, int* err, int ksplit, float* __restrict__ part_out,
    int* __restrict__ route_counts) {
  __shared__ float part[kRouteWaves][kRouteChunk][65];
  __shared__ int cnt[64];
  __shared__ int last;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Raised issue priority: on a two-stream forward this launch shares CUs
  // with the shared expert's GEMM, whose waves would otherwise take turns
  // with it on every SIMD.
  __builtin_amdgcn_s_setprio(3);
  const int chunk = blockIdx.x / ksplit, p = blockIdx.x % ksplit;
  const int t0 = chunk * kRouteChunk;
  if (tid < 64) cnt[tid] = 0;
  const int ar = lane & 15;        // fragment row (token) / column (expert)
  const int aq = (lane >> 4) * 8;  // fragment k offset within a 32-wide step
  const int steps = H / 32;
  // Range-checked buffer loads: tokens >= T and experts >= E read as zero.
  // The x range starts at this workgroup's first token so offsets stay small.
  const int nt = min(kRouteChunk, T - t0);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(x + (size_t)t0 * H), 0, (int)((uint32_t)nt * H * 4u), 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(w), 0, (int)((uint32_t)E * H * 2u), 0x00020000);
  constexpr uint32_t kFar = 0x80000000u;
  const uint32_t xoff = (uint32_t)ar * H * 4u + aq * 4u;
  u32x4 xa[KS], xb[KS], wv[KS][4];
  auto step_of = [&](int i) { return p + ksplit * (wave + kRouteWaves * i); };
#pragma unroll
  for (int i = 0; i < KS; i++) {
    const int st = step_of(i);
    const bool ok = st < steps;
    const uint32_t k0 = (uint32_t)st * 32u;
    xa[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? xoff + k0 * 4u : kFar, 0, 0);
    xb[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? xoff + k0 * 4u + 16u : kFar, 0, 0);
#pragma unroll
    for (int ni = 0; ni < 4; ni++) {
      const uint32_t e = (uint32_t)(ni * 16 + ar);
      wv[i][ni] = __builtin_amdgcn_raw_buffer_load_b128(
          wr, ok ? (e * H + k0 + aq) * 2u : kFar, 0, 0);
    }
  }
  floatx4 acc[4];
#pragma unroll
  for (int ni = 0; ni < 4; ni++) acc[ni] = floatx4{0.f, 0.f, 0.f, 0.f};
  // The grouped GEMM's input planes (x_hi set): hi = bf16(x), lo = bf16(x
  // - hi), the first two of the three terms below, k-blocked ([H/32][T][32]:
  // step st of token t at (st T + t) 32), through a resource over the whole
  // plane; tokens past T and steps past H / 32 store nothing.
  const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
      x_hi, 0, (int)((uint32_t)T * H * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t lr = __builtin_amdgcn_make_buffer_rsrc(
      x_lo, 0, (int)((uint32_t)T * H * 2u), 0x00020000);
#pragma unroll
  for (int i = 0; i < KS; i++) {
    const float xv[8] = {__uint_as_float(xa[i].x), __uint_as_float(xa[i].y),
                         __uint_as_float(xa[i].z), __uint_as_float(xa[i].w),
                         __uint_as_float(xb[i].x), __uint_as_float(xb[i].y),
                         __uint_as_float(xb[i].z), __uint_as_float(xb[i].w)};
    bf16x8 hi, mid, lo;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float f = xv[j];
      const __bf16 h = (__bf16)f;
      const float r1 = f - (float)h;
      const __bf16 m = (__bf16)r1;
      hi[j] = h;
      mid[j] = m;
      lo[j] = (__bf16)(r1 - (float)m);
    }
    if (x_hi) {
      const int st = step_of(i);
      int off = st < steps && ar < nt
                    ? (int)((((uint32_t)st * T + (uint32_t)(t0 + ar)) * 32u + aq) * 2u)
                    : (int)kFar;
      asm volatile("" : "+v"(off));  // the whole offset in the range-checked VGPR field
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hi), hr, off, 0, 0);
      if (x_lo) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, mid), lr, off, 0, 0);
    }
#pragma unroll
    for (int ni = 0; ni < 4; ni++) {
      const bf16x8 bb = __builtin_bit_cast(bf16x8, wv[i][ni]);
      acc[ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, bb, acc[ni], 0, 0, 0);
      acc[ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mid, bb, acc[ni], 0, 0, 0);
      acc[ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, bb, acc[ni], 0, 0, 0);
    }
  }
  // acc[ni][r]: token 4 (lane / 16) + r, expert 16 ni + lane % 16.
#pragma unroll
  for (int ni = 0; ni < 4; ni++)
#pragma unroll
    for (int r = 0; r < 4; r++) part[wave][4 * (lane >> 4) + r][ni * 16 + ar] = acc[ni][r];
  __syncthreads();
  // Wave partial sums in wave order (deterministic).
  auto wave_sum_of = [&](int tl, int e) {
    float v = part[0][tl][e];
#pragma unroll
    for (int q = 1; q < kRouteWaves; q++) v = v + part[q][tl][e];
    return v;
  };
  constexpr int kPer = kRouteChunk / kRouteWaves;
  if (ksplit > 1) {
    float* out = part_out + (size_t)blockIdx.x * kRouteChunk * 64;
    float mine[kPer];
#pragma unroll
    for (int j = 0; j < kPer; j++) {
      const int tl = wave * kPer + j;
      mine[j] = wave_sum_of(tl, lane);
      __hip_atomic_store(out + tl * 64 + lane, mine[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partials are complete
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(route_counts + chunk * 16, 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == ksplit - 1;
    __syncthreads();
    if (!last) return;
    if (tid == 0) __hip_atomic_store(route_counts + chunk * 16, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Every partial of the chunk, loaded before the first add, then added
    // in workgroup order (this workgroup's own from registers).
    const float* in = part_out + (size_t)chunk * ksplit * kRouteChunk * 64;
    float v[kPer][kMaxRouteSplit];
#pragma unroll
    for (int j = 0; j < kPer; j++)
#pragma unroll
      for (int q = 0; q < kMaxRouteSplit; q++)
        v[j][q] = q < ksplit && q != p
                      ? __hip_atomic_load(in + ((size_t)q * kRouteChunk + wave * kPer + j) * 64 + lane,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : mine[j];
#pragma unroll
    for (int j = 0; j < kPer; j++) {
      float a = v[j][0];
#pragma unroll
      for (int q = 1; q < kMaxRouteSplit; q++)
        if (q < ksplit) a = a + v[j][q];
      part[0][wave * kPer + j][lane] = a;
    }
    __syncthreads();
    route_chunk([&](int tl, int e) { return part[0][tl][e]; }, chunk, T, E, K, normalize, scale,
                logits, ids, weights, chunk_counts, cnt, err);
    return;
  }
  // Each wave routes two tokens on its own with the wave top-k.
  route_chunk(wave_sum_of, chunk, T, E, K, normalize, scale, logits, ids, weights, chunk_counts, cnt,
              err);
}


void launch_router_topk_mfma(const float* x, const uint16_t* w, int T, int H, int E, int K,
                             int normalize, float scale, float* logits, int* ids, float* weights,
                             int* chunk_counts, uint16_t* x_hi, uint16_t* x_lo, int* err,
                             float* part, int* route_counts, hipStream_t s) {
  if (T <= 0 || !router_mfma_supported(H)) return;
  const int chunks = (T + kRouteChunk - 1) / kRouteChunk;
  const int ksplit = part && route_counts ? router_ksplit(T, H) : 1;
  const dim3 grid(chunks * ksplit), block(64 * kRouteWaves);
  const int steps = H / 32;
  const int ks = (steps + ksplit * kRouteWaves - 1) / (ksplit * kRouteWaves);
  if (ks <= 1)
    router_mfma_kernel<1><<<grid, block, 0, s>>>(x, w, T, H, E, K, normalize, scale, logits, ids,
                                                 weights, chunk_counts, x_hi, x_lo, err, ksplit, part,
                                                 route_counts);
  else if (ks <= 5)
    router_mfma_kernel<5><<<grid, block, 0, s>>>(x, w, T, H, E, K, normalize, scale, logits, ids,
                                                 weights, chunk_counts, x_hi, x_lo, err, ksplit, part,
                                                 route_counts);
  else
    router_mfma_kernel<8><<<grid, block, 0, s>>>(x, w, T, H, E, K, normalize, scale, logits, ids,
                                                 weights, chunk_counts, x_hi, x_lo, err, ksplit, part,
                                                 route_counts);
}

void launch_topk(const float* logits, int T, int n, int K, int normalize, float scale, int* ids,
                 float* weights, int* err, hipStream_t s) {
  if (T <= 0) return;
  hipLaunchKernelGGL(topk_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, n, K, normalize,
                     scale, ids, weights, err);
}

}  // namespace uocr
