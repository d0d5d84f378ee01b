// One-token (decode) expert engine: bound by the bytes of the active
// experts' weights, so every workgroup is one wave over 8 weight rows that
// issues all of its weight (and scale) loads before using any of them.
//
// Arithmetic is that of Decoder::projection / feed_forward for one row
// (src/decoder/mod.rs:99-122): BF16 widened exactly; INT8 weight-only as
// the rounded product w * scale (src/cpu/quantized.rs:119-131); W8A8 for
// DynamicActivations (one row is always a single-row group, :103-104) with
// the row quantised per 32-block and exact i32 block sums (:155-236).
//
// Gate/up writes the raw gate and up values (interleaved row order of w13);
// down builds h = silu(g) * u while staging it into LDS, then the last
// workgroup of each 8-feature block adds the block's contributions in the
// reference order (shared first, experts ascending, mul then add).
#include "common.hpp"
#include "moe_kernels.hpp"

namespace uocr {

namespace {

enum { kBF16 = 0, kInt8 = 1, kW8A8 = 2 };
constexpr int kRows = 8;     // weight rows per workgroup (one wave)
constexpr int kLpr = 16;     // lanes per row
constexpr int kMaxC = 14;    // 16-byte chunks per lane per row: K <= 1792 (bf16) / 3584 (int8)
constexpr int kKmax = 1792;  // widest activation row (LDS)

// Quantise an FP32 row held in LDS per 32-block (Int8Matrix::quantize,
// src/cpu/quantized.rs:43-74); non-finite input or an underflowing scale
// raises Numerical.
__device__ void quantize_lds(const float* xl, int K, int8_t* xq, float* xs, int* err) {
  for (int b = threadIdx.x; b < K / kQBlock; b += blockDim.x) {
    const float* v = xl + b * kQBlock;
    float maximum = 0.0f;
    bool bad = false;
    for (int i = 0; i < kQBlock; i++) {
      bad |= !isfinite(v[i]);
      maximum = fmaxf(maximum, fabsf(v[i]));
    }
    const float scale = maximum / 127.0f;
    if (bad || (maximum > 0.0f && scale == 0.0f)) raise_error(err, kErrNumerical);
    xs[b] = scale;
    for (int i = 0; i < kQBlock; i++) {
      int q = 0;
      if (scale != 0.0f) q = (int)fminf(fmaxf(rintf(v[i] / scale), -127.0f), 127.0f);
      xq[b * kQBlock + i] = (int8_t)q;
    }
  }
}

// Dots rows [row0, row0 + 8) of a [rows_total, K] matrix with the LDS row
// (xl, or xq/xs for W8A8). Lane mapping: 16 lanes per row (q = lane / 16
// picks the row within an iteration of 4), lane j = lane % 16 takes chunks
// j, j + 16, ... Returns this lane's row sum in out_lane for rows
// row0 + q and row0 + 4 + q (valid in lanes with j == 0).
template <int KIND>
__device__ __forceinline__ void dot8(const void* __restrict__ wbase, const float* __restrict__ sbase,
                                     int K, int rows_total, int row0, const float* xl,
                                     const int8_t* xq, const float* xs, float& r0, float& r1) {
  constexpr int kElems = KIND == kBF16 ? 8 : 16;
  constexpr int kBytes = KIND == kBF16 ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15;
  const int nchunks = K / kElems;
  const int nblk = K / kQBlock;
  const int ra = row0 + q, rb = row0 + 4 + q;
  const int ca = ra < rows_total ? ra : 0, cb = rb < rows_total ? rb : 0;
  const uint4* wa = reinterpret_cast<const uint4*>(static_cast<const char*>(wbase) +
                                                   (size_t)ca * K * kBytes);
  const uint4* wb = reinterpret_cast<const uint4*>(static_cast<const char*>(wbase) +
                                                   (size_t)cb * K * kBytes);
  // Every load first (exec-masked past the row, no selects on the loaded
  // values), so all of them are in flight before the first is used.
  uint4 va[kMaxC], vb[kMaxC];
  float sa[kMaxC], sb[kMaxC];
#pragma unroll
  for (int m = 0; m < kMaxC; m++) {
    const int c = j + kLpr * m;
    if (c < nchunks) {
      va[m] = wa[c];
      vb[m] = wb[c];
      if constexpr (KIND != kBF16) {
        sa[m] = sbase[(size_t)ca * nblk + (c >> 1)];
        sb[m] = sbase[(size_t)cb * nblk + (c >> 1)];
      }
    }
  }
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int m = 0; m < kMaxC; m++) {
    const int c = j + kLpr * m;
    if (c >= nchunks) break;
    if constexpr (KIND == kBF16) {
      const float4* xp = reinterpret_cast<const float4*>(xl + c * 8);
      const float4 x0 = xp[0], x1 = xp[1];
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      const uint32_t ua[4] = {va[m].x, va[m].y, va[m].z, va[m].w};
      const uint32_t ub[4] = {vb[m].x, vb[m].y, vb[m].z, vb[m].w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        a0 = fmaf(bf16_lo(ua[i]), xv[2 * i], a0);
        a0 = fmaf(bf16_hi(ua[i]), xv[2 * i + 1], a0);
        a1 = fmaf(bf16_lo(ub[i]), xv[2 * i], a1);
        a1 = fmaf(bf16_hi(ub[i]), xv[2 * i + 1], a1);
      }
    } else if constexpr (KIND == kInt8) {
      const uint32_t ua[4] = {va[m].x, va[m].y, va[m].z, va[m].w};
      const uint32_t ub[4] = {vb[m].x, vb[m].y, vb[m].z, vb[m].w};
      const float4* xp = reinterpret_cast<const float4*>(xl + c * 16);
#pragma unroll
      for (int v4 = 0; v4 < 4; v4++) {
        const float4 xv = xp[v4];
        const float xs4[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const float da = (float)(int8_t)((ua[v4] >> (8 * b)) & 0xff) * sa[m];
          const float db = (float)(int8_t)((ub[v4] >> (8 * b)) & 0xff) * sb[m];
          a0 = fmaf(da, xs4[b], a0);
          a1 = fmaf(db, xs4[b], a1);
        }
      }
    } else {
      const int4 xv = *reinterpret_cast<const int4*>(xq + c * 16);
      int pa = __builtin_amdgcn_sdot4((int)va[m].x, xv.x, 0, false);
      pa = __builtin_amdgcn_sdot4((int)va[m].y, xv.y, pa, false);
      pa = __builtin_amdgcn_sdot4((int)va[m].z, xv.z, pa, false);
      pa = __builtin_amdgcn_sdot4((int)va[m].w, xv.w, pa, false);
      int pb = __builtin_amdgcn_sdot4((int)vb[m].x, xv.x, 0, false);
      pb = __builtin_amdgcn_sdot4((int)vb[m].y, xv.y, pb, false);
      pb = __builtin_amdgcn_sdot4((int)vb[m].z, xv.z, pb, false);
      pb = __builtin_amdgcn_sdot4((int)vb[m].w, xv.w, pb, false);
      // Chunks 2b and 2b+1 (lanes j, j^1) form block b: exact i32 sum.
      const int sa_i = pa + __shfl_xor(pa, 1);
      const int sb_i = pb + __shfl_xor(pb, 1);
      if ((j & 1) == 0) {
        const int b = c >> 1;
        a0 += (float)sa_i * sa[m] * xs[b];
        a1 += (float)sb_i * sb[m] * xs[b];
      }
    }
  }
  r0 = group16_sum(a0);
  r1 = group16_sum(a1);
}

template <int KIND>
__global__ __launch_bounds__(64) void decode_gateup_kernel(DeviceLayer L, Scratch S) {
  __shared__ __align__(16) float xl[kKmax];
  __shared__ __align__(16) int8_t xq[kKmax];
  __shared__ float xs[kKmax / kQBlock];
  const int tile = blockIdx.y;
  if (tile >= S.counters[0]) return;
  const int g = S.tiles[2 * tile];
  const int W = L.width(g);
  const int row0 = blockIdx.x * kRows;
  if (row0 >= 2 * W) return;
  const bool routed = g < L.E;
  const int token = routed ? S.perm_rows[S.offsets[g]] : 0;
  const float* x = S.xn + (size_t)token * L.H;
  {
    // All activation loads in flight at once (H <= kKmax).
    constexpr int kV = kKmax / 4 / 64;
    float4 v[kV];
#pragma unroll
    for (int i = 0; i < kV; i++) {
      const int at = threadIdx.x + 64 * i;
      if (at < L.H / 4) v[i] = reinterpret_cast<const float4*>(x)[at];
    }
#pragma unroll
    for (int i = 0; i < kV; i++) {
      const int at = threadIdx.x + 64 * i;
      if (at < L.H / 4) reinterpret_cast<float4*>(xl)[at] = v[i];
    }
  }
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    quantize_lds(xl, L.H, xq, xs, S.err);
    __syncthreads();
  }
  const void* w = KIND == kBF16 ? (const void*)(L.w13 + L.w13_offset(g))
                                : (const void*)(L.q13 + L.w13_offset(g));
  const float* sc = KIND == kBF16 ? nullptr : L.s13 + L.s13_offset(g);
  float r0, r1;
  dot8<KIND>(w, sc, L.H, 2 * W, row0, xl, xq, xs, r0, r1);
  const int lane = threadIdx.x;
  if ((lane & 15) == 0) {
    // gu holds, per group, its 2W gate/up values in w13 row order.
    float* gu = S.gu + (routed ? (size_t)S.offsets[g] * 2 * L.I : (size_t)S.offsets[L.E] * 2 * L.I);
    const int ra = row0 + (lane >> 4), rb = ra + 4;
    if (ra < 2 * W) gu[ra] = r0;
    if (rb < 2 * W) gu[rb] = r1;
  }
}

template <int KIND>
__global__ __launch_bounds__(64) void decode_down_kernel(DeviceLayer L, Scratch S,
                                                         const float* residual, float* out) {
  __shared__ __align__(16) float hl[kKmax];
  __shared__ __align__(16) int8_t hq[kKmax];
  __shared__ float hs[kKmax / kQBlock];
  __shared__ int ticket;
  const int ntiles = S.counters[0];
  const int tile = blockIdx.y;
  if (tile >= ntiles) return;
  const int g = S.tiles[2 * tile];
  const int W = L.width(g);
  const int row0 = blockIdx.x * kRows;  // output features
  const bool routed = g < L.E;
  const float* gu = S.gu + (routed ? (size_t)S.offsets[g] * 2 * L.I
                                   : (size_t)S.offsets[L.E] * 2 * L.I);
  // h[k] = silu(gate_k) * up_k; gate k and up k sit 32 rows apart in each
  // 64-row block of the interleaved order. Lane l takes the 4-value groups
  // l, l + 64, ... of the gate half; every load is issued before any use.
  {
    constexpr int kV = kKmax / 4 / 64;
    float4 gv[kV], uv[kV];
#pragma unroll
    for (int i = 0; i < kV; i++) {
      const int grp = threadIdx.x + 64 * i;  // 4 hidden values per group
      if (grp * 4 < W) {
        const int k = grp * 4, blk = k >> 5, o = k & 31;
        gv[i] = *reinterpret_cast<const float4*>(gu + blk * 64 + o);
        uv[i] = *reinterpret_cast<const float4*>(gu + blk * 64 + 32 + o);
      }
    }
#pragma unroll
    for (int i = 0; i < kV; i++) {
      const int grp = threadIdx.x + 64 * i;
      if (grp * 4 < W) {
        float4 h;
        h.x = silu(gv[i].x) * uv[i].x;
        h.y = silu(gv[i].y) * uv[i].y;
        h.z = silu(gv[i].z) * uv[i].z;
        h.w = silu(gv[i].w) * uv[i].w;
        *reinterpret_cast<float4*>(hl + grp * 4) = h;
      }
    }
  }
  __syncthreads();
  if constexpr (KIND == kW8A8) {
    quantize_lds(hl, W, hq, hs, S.err);
    __syncthreads();
  }
  const void* w = KIND == kBF16 ? (const void*)(L.w2 + L.w2_offset(g))
                                : (const void*)(L.q2 + L.w2_offset(g));
  const float* sc = KIND == kBF16 ? nullptr : L.s2 + L.s2_offset(g);
  float r0, r1;
  dot8<KIND>(w, sc, W, L.H, row0, hl, hq, hs, r0, r1);
  const int lane = threadIdx.x;
  if ((lane & 15) == 0) {
    float* yrow = routed ? S.y + (size_t)S.offsets[g] * L.H : S.ys;
    const int fa = row0 + (lane >> 4), fb = fa + 4;
    if (fa < L.H) yrow[fa] = r0;
    if (fb < L.H) yrow[fb] = r1;
  }
  // Last workgroup of this feature block: ordered combine.
  __threadfence();
  __syncthreads();
  if (lane == 0) ticket = atomicAdd(&S.sync[kSyncDown + blockIdx.x], 1);
  __syncthreads();
  if (ticket != ntiles - 1) return;
  __threadfence();
  if (lane == 0) atomicExch(&S.sync[kSyncDown + blockIdx.x], 0);
  if (lane < kRows) {
    const int f = row0 + lane;
    if (f < L.H) {
      const int K = L.K;
      int e[8], pos[8];
      float p[8];
      for (int jj = 0; jj < K; jj++) {
        e[jj] = S.topk_ids[jj];
        pos[jj] = S.inv_pos[jj];
        p[jj] = S.topk_w[jj];
        for (int b = jj; b > 0 && e[b] < e[b - 1]; b--) {
          int te = e[b]; e[b] = e[b - 1]; e[b - 1] = te;
          int tp = pos[b]; pos[b] = pos[b - 1]; pos[b - 1] = tp;
          float tw = p[b]; p[b] = p[b - 1]; p[b - 1] = tw;
        }
      }
      float acc = S.ys[f];
      for (int jj = 0; jj < K; jj++) acc = acc + p[jj] * S.y[(size_t)pos[jj] * L.H + f];
      if (residual) acc = residual[f] + acc;
      out[f] = acc;
    }
  }
}

}  // namespace

bool decode_supported(const DeviceLayer& L) {
  // LDS rows of kKmax floats; one election counter per 8-feature block.
  const int kmax = L.H > L.S ? L.H : L.S;
  return kmax <= kKmax && L.H <= 2048 && L.H / kRows <= kSyncSize - kSyncDown;
}

void launch_decode_gateup(const DeviceLayer& L, const Scratch& S, int tiles_bound,
                          hipStream_t s) {
  const dim3 grid((2 * L.S + kRows - 1) / kRows, tiles_bound);
  if (L.quant_mode == 0)
    decode_gateup_kernel<kBF16><<<grid, dim3(64), 0, s>>>(L, S);
  else if (L.quant_mode == 1)
    decode_gateup_kernel<kInt8><<<grid, dim3(64), 0, s>>>(L, S);
  else
    decode_gateup_kernel<kW8A8><<<grid, dim3(64), 0, s>>>(L, S);
}

void launch_decode_down(const DeviceLayer& L, const Scratch& S, int tiles_bound,
                        const float* residual, float* out, hipStream_t s) {
  const dim3 grid((L.H + kRows - 1) / kRows, tiles_bound);
  if (L.quant_mode == 0)
    decode_down_kernel<kBF16><<<grid, dim3(64), 0, s>>>(L, S, residual, out);
  else if (L.quant_mode == 1)
    decode_down_kernel<kInt8><<<grid, dim3(64), 0, s>>>(L, S, residual, out);
  else
    decode_down_kernel<kW8A8><<<grid, dim3(64), 0, s>>>(L, S, residual, out);
}

}  // namespace uocr
