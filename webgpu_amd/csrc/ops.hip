// ops.hip — RMSNorm, RoPE (Q/K-norm + half-split, half-split, adjacent), residual add,
// SwiGLU / GeGLU, bias, SiLU, KV ring append and greedy argmax for gfx950.
//
// Semantics follow src/core/shaders.ts: normShader :55-68, ropeShader :69-87,
// ropeNeoxShader :139-152, ropeClassicShader :155-168, addShader :123-128,
// geluShader :129-137, biasAddShader :170-175, activateShader :177-181, siluShader
// (src/core/qwen-shaders.ts:27-34), the KV copies of engine.ts:120-124 / context.ts:34-37
// and sample(T=0) of engine.ts:305-309. RoPE angles are formed in f64
// (pos * scale * theta^(-2i/rot)) with f64 sin/cos so long positions track the f64 oracle.
#include "internal.h"
#include "decode.h"
#include "split.h"
#include "matvec.h"

namespace wgd {

// ------------------------------------------------------------------ block reduction
__device__ __forceinline__ float block_sum_256(float v, float *red) {
  v = wave_sum(v);
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// ------------------------------------------------------------------ RMSNorm
__global__ __launch_bounds__(256) void k_norm(const float *x, const float *w, float *y, uint32_t n, float eps) {
  __shared__ float red[4];
  const float *xr = x + (uint64_t)blockIdx.x * n;
  float *yr = y + (uint64_t)blockIdx.x * n;
  float s = 0.f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) { float v = xr[i]; s += v * v; }
  s = block_sum_256(s, red);
  float inv = 1.f / sqrtf(s / (float)n + eps);
  for (uint32_t i = threadIdx.x; i < n; i += 256) yr[i] = xr[i] * inv * w[i];
}

hipError_t norm(hipStream_t s, const float *x, const float *w, float *y, uint32_t n, float eps, uint32_t batch) {
  if (!batch || !n) return hipSuccess;
  hipLaunchKernelGGL(k_norm, dim3(batch), dim3(256), 0, s, x, w, y, n, eps);
  return hipGetLastError();
}

// One token per workgroup, eight consecutive elements per thread step: the f32 output and
// its split form for the GEMMs that read it.
__global__ __launch_bounds__(256) void k_norm_split(const float *x, const float *w, float *y, uint16_t *xs,
                                                    uint32_t n, float eps) {
  __shared__ float red[4];
  const uint32_t tok = blockIdx.x;
  const float *xr = x + (uint64_t)tok * n;
  float *yr = y + (uint64_t)tok * n;
  float s = 0.f;
  for (uint32_t k = 8 * threadIdx.x; k < n; k += 8 * 256) {
    const float4 a = *(const float4 *)(xr + k), b = *(const float4 *)(xr + k + 4);
    s += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w;
  }
  s = block_sum_256(s, red);
  const float inv = 1.f / sqrtf(s / (float)n + eps);
  for (uint32_t k = 8 * threadIdx.x; k < n; k += 8 * 256) {
    float4 a = *(const float4 *)(xr + k), b = *(const float4 *)(xr + k + 4);
    const float4 wa = *(const float4 *)(w + k), wb = *(const float4 *)(w + k + 4);
    a = make_float4(a.x * inv * wa.x, a.y * inv * wa.y, a.z * inv * wa.z, a.w * inv * wa.w);
    b = make_float4(b.x * inv * wb.x, b.y * inv * wb.y, b.z * inv * wb.z, b.w * inv * wb.w);
    *(float4 *)(yr + k) = a;
    *(float4 *)(yr + k + 4) = b;
    split_store8(xs, n, tok, k, a, b);
  }
}

// The finish of a residual projection (O or down) kept as split-K partials, fused with the
// RMSNorm that reads the residual next: per token, state += the partials summed in split
// order, then y = RMSNorm(state) * w and its split form xs. With post_w (Gemma's post-norms)
// the summed partials are a delta that enters as RMSNorm(delta) * post_w. One 512-thread
// workgroup per token, eight consecutive elements per thread step (n <= RN_G * 8 * 512).
constexpr uint32_t RN_T = 512, RN_G = 4;
// The sum over the workgroup of each thread's ss, in a fixed order.
__device__ __forceinline__ float block_total(float ss, float *red) {
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  ss = wave_sum(ss);
  __syncthreads();  // red is free again
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (uint32_t u = 0; u < RN_T / 64; u++) ss += red[u];
  return ss;
}
__global__ __launch_bounds__(512) void k_reduce_norm_split(const float *part, uint32_t splits, float *state,
                                                           const float *post_w, const float *w, float *y,
                                                           uint16_t *xs, uint32_t n, uint32_t batch, float eps) {
  __shared__ float red[RN_T / 64];
  const uint32_t tok = blockIdx.x, tid = threadIdx.x;
  const uint64_t stride = (uint64_t)n * batch;
  const __amdgpu_buffer_rsrc_t rp = split_rsrc(part, splits, stride);
  float *sr = state + (uint64_t)tok * n;
  float v[RN_G][8];
  float ss = 0.f;
#pragma unroll
  for (uint32_t gi = 0; gi < RN_G; gi++) {
    const uint32_t k = 8 * (tid + RN_T * gi);
    if (k >= n) break;  // uniform per thread
    const uint32_t off = 4 * (tok * n + k);
    const float4 a = split_sum4<MAX_SPLITS>(rp, splits, (uint32_t)(4 * stride), off);
    const float4 b = split_sum4<MAX_SPLITS>(rp, splits, (uint32_t)(4 * stride), off + 16);
    v[gi][0] = a.x; v[gi][1] = a.y; v[gi][2] = a.z; v[gi][3] = a.w;
    v[gi][4] = b.x; v[gi][5] = b.y; v[gi][6] = b.z; v[gi][7] = b.w;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += v[gi][e] * v[gi][e];
  }
  // the delta's norm factor (post_w), then state += delta (times it and post_w)
  const float dinv = post_w ? 1.f / sqrtf(block_total(ss, red) / (float)n + eps) : 1.f;
  ss = 0.f;
#pragma unroll
  for (uint32_t gi = 0; gi < RN_G; gi++) {
    const uint32_t k = 8 * (tid + RN_T * gi);
    if (k >= n) break;
    const float4 ha = *(const float4 *)(sr + k), hb = *(const float4 *)(sr + k + 4);
    const float h[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
    if (post_w) {
      const float4 pa = *(const float4 *)(post_w + k), pb = *(const float4 *)(post_w + k + 4);
      const float pw[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
      for (int e = 0; e < 8; e++) v[gi][e] = h[e] + v[gi][e] * dinv * pw[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) v[gi][e] = h[e] + v[gi][e];
    }
    *(float4 *)(sr + k) = make_float4(v[gi][0], v[gi][1], v[gi][2], v[gi][3]);
    *(float4 *)(sr + k + 4) = make_float4(v[gi][4], v[gi][5], v[gi][6], v[gi][7]);
#pragma unroll
    for (int e = 0; e < 8; e++) ss += v[gi][e] * v[gi][e];
  }
  const float inv = 1.f / sqrtf(block_total(ss, red) / (float)n + eps);
  float *yr = y + (uint64_t)tok * n;
#pragma unroll
  for (uint32_t gi = 0; gi < RN_G; gi++) {
    const uint32_t k = 8 * (tid + RN_T * gi);
    if (k >= n) break;
    const float4 wa = *(const float4 *)(w + k), wb = *(const float4 *)(w + k + 4);
    const float4 a = make_float4(v[gi][0] * inv * wa.x, v[gi][1] * inv * wa.y, v[gi][2] * inv * wa.z, v[gi][3] * inv * wa.w);
    const float4 b = make_float4(v[gi][4] * inv * wb.x, v[gi][5] * inv * wb.y, v[gi][6] * inv * wb.z, v[gi][7] * inv * wb.w);
    *(float4 *)(yr + k) = a;
    *(float4 *)(yr + k + 4) = b;
    split_store8(xs, n, tok, k, a, b);
  }
}

// The deferred-norm finish of a residual projection: one 128-thread workgroup per token and
// segment, eight elements per thread a step, so the partials stream over every CU; each
// segment's sum of squares goes to sq (each thread's elements in order, the DPP fold of
// each wavefront, then the two wavefronts in order).
//
// The segments follow the split-K GEMM that wrote the partials. Its 128-row tile t ran on
// XCD t % 8 (its grid's first dimension is the tile count, a multiple of 8 here, and
// workgroups are dispatched to the XCDs round-robin). So when n is a multiple of 1024,
// segment x holds the tiles t = x (mod 8), and workgroup (x, token), dispatched to XCD x,
// reads only partials that XCD wrote. Each 128-row run of the scratch then stays with one
// XCD, so the next GEMM's writes to it find no copy in another XCD's L2 to invalidate
// (coherence probes, which slow that GEMM). Otherwise segment x is elements
// [RS_E x, RS_E (x + 1)).
constexpr uint32_t RS_T = 128, RS_E = 8 * RS_T;
static bool residual_by_xcd(uint32_t n) { return n % 1024 == 0; }
uint32_t residual_split_segs(uint32_t n) { return residual_by_xcd(n) ? 8 : (n + RS_E - 1) / RS_E; }
__global__ __launch_bounds__(128) void k_residual_split(const float *part, uint32_t splits, float *state,
                                                        const float *w, uint16_t *xs, float *sq, uint32_t n,
                                                        uint32_t batch, uint32_t by_xcd) {
  __shared__ float red[RS_T / 64];
  const uint32_t seg = blockIdx.x, tok = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t stride = (uint64_t)n * batch;
  const __amdgpu_buffer_rsrc_t rp = split_rsrc(part, splits, stride);
  // this thread's groups of eight: group j of the segment starts at element col(j)
  const uint32_t groups = by_xcd ? n / 64 : (seg * RS_E + RS_E <= n ? RS_E : n - seg * RS_E) / 8;
  auto col = [&](uint32_t j) { return by_xcd ? (seg + 8 * (j / 16)) * 128 + (j % 16) * 8 : seg * RS_E + 8 * j; };
  float ss = 0.f;
  for (uint32_t j = tid; j < groups; j += RS_T) {
    const uint32_t k = col(j);
    float *sr = state + (uint64_t)tok * n + k;
    const uint32_t off = 4 * (tok * n + k);
    float4 a = split_sum4<MAX_SPLITS>(rp, splits, (uint32_t)(4 * stride), off);
    float4 b = split_sum4<MAX_SPLITS>(rp, splits, (uint32_t)(4 * stride), off + 16);
    const float4 ha = *(const float4 *)sr, hb = *(const float4 *)(sr + 4);
    a = make_float4(ha.x + a.x, ha.y + a.y, ha.z + a.z, ha.w + a.w);
    b = make_float4(hb.x + b.x, hb.y + b.y, hb.z + b.z, hb.w + b.w);
    *(float4 *)sr = a;
    *(float4 *)(sr + 4) = b;
    ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w;
    const float4 wa = *(const float4 *)(w + k), wb = *(const float4 *)(w + k + 4);
    split_store8(xs, n, tok, k, make_float4(a.x * wa.x, a.y * wa.y, a.z * wa.z, a.w * wa.w),
                 make_float4(b.x * wb.x, b.y * wb.y, b.z * wb.z, b.w * wb.w));
  }
  ss = wave_total(ss);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  if (tid == 0) sq[(uint64_t)tok * gridDim.x + seg] = red[0] + red[1];
}

hipError_t residual_split(hipStream_t s, const float *part, uint32_t splits, float *state, const float *w, uint16_t *xs,
                          float *sq, uint32_t n, uint32_t batch) {
  if (!batch) return hipSuccess;
  if (n % SPLIT_K || !splits || splits > MAX_SPLITS || (uint64_t)splits * n * batch * 4 >= (1ull << 31) || !sq ||
      ((uintptr_t)part | (uintptr_t)state | (uintptr_t)w) % 16)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_residual_split, dim3(residual_split_segs(n), batch), dim3(RS_T), 0, s, part, splits, state, w,
                     xs, sq, n, batch, residual_by_xcd(n) ? 1u : 0u);
  return hipGetLastError();
}

hipError_t reduce_norm_split(hipStream_t s, const float *part, uint32_t splits, float *state, const float *w, float *y,
                             uint16_t *xs, uint32_t n, float eps, uint32_t batch, const float *post_w) {
  if (!batch) return hipSuccess;
  if (n % SPLIT_K || n > RN_G * 8 * RN_T || !splits || splits > MAX_SPLITS ||
      (uint64_t)splits * n * batch * 4 >= (1ull << 31) ||
      ((uintptr_t)part | (uintptr_t)state | (uintptr_t)w | (uintptr_t)y | (uintptr_t)post_w) % 16)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_reduce_norm_split, dim3(batch), dim3(RN_T), 0, s, part, splits, state, post_w, w, y, xs, n,
                     batch, eps);
  return hipGetLastError();
}

hipError_t norm_split(hipStream_t s, const float *x, const float *w, float *y, uint16_t *xs, uint32_t n, float eps,
                      uint32_t batch) {
  if (!batch) return hipSuccess;
  if (n % SPLIT_K || ((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) % 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_norm_split, dim3(batch), dim3(256), 0, s, x, w, y, xs, n, eps);
  return hipGetLastError();
}

// state += norm(delta) * w (Gemma 3 post-attention / post-FFN norms, engine.ts:165-166,172-173)
__global__ __launch_bounds__(256) void k_norm_add(const float *d, const float *w, float *state, uint32_t n, float eps) {
  __shared__ float red[4];
  const float *dr = d + (uint64_t)blockIdx.x * n;
  float *sr = state + (uint64_t)blockIdx.x * n;
  float s = 0.f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) { float v = dr[i]; s += v * v; }
  s = block_sum_256(s, red);
  float inv = 1.f / sqrtf(s / (float)n + eps);
  for (uint32_t i = threadIdx.x; i < n; i += 256) sr[i] += dr[i] * inv * w[i];
}

// The same for rows of up to NA_T * NA_E elements: one 1024-thread workgroup per row with
// every element loaded at once (the strided loop above is a chain of dependent round trips
// at batch 1). With q.d0 set it also writes the QX form of the new state times next_w, the
// input of the next projection with its RMSNorm pending (elements i + NA_T e: each 16-lane
// group holds 16 consecutive elements).
constexpr uint32_t NA_T = 1024, NA_E = 12;
__global__ __launch_bounds__(1024) void k_norm_add_q(const float *d, const float *w, float *state, uint32_t n,
                                                     float eps, const float *next_w, QXOut q) {
  __shared__ float red[NA_T / 64];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float *dr = d + (uint64_t)blockIdx.x * n;
  float *sr = state + (uint64_t)blockIdx.x * n;
  // every load goes out before the reduction: one round trip per launch
  float dv[NA_E], sv[NA_E], wv_[NA_E], nw[NA_E], s = 0.f;
#pragma unroll
  for (uint32_t e = 0; e < NA_E; e++) {
    const uint32_t i = tid + NA_T * e;
    const bool live = i < n;
    dv[e] = live ? dr[i] : 0.f;
    sv[e] = live ? sr[i] : 0.f;
    wv_[e] = live ? w[i] : 0.f;
    nw[e] = live && next_w ? next_w[i] : 0.f;
  }
#pragma unroll
  for (uint32_t e = 0; e < NA_E; e++) s += dv[e] * dv[e];
  s = wave_sum(s);
  if (lane == 0) red[wv] = s;
  __syncthreads();
  s = 0.f;
#pragma unroll
  for (uint32_t u = 0; u < NA_T / 64; u++) s += red[u];
  const float inv = 1.f / sqrtf(s / (float)n + eps);
#pragma unroll
  for (uint32_t e = 0; e < NA_E; e++) {
    const uint32_t i = tid + NA_T * e;
    if (NA_T * e >= n) break;  // uniform
    const bool live = i < n;
    const float nv = live ? sv[e] + dv[e] * inv * wv_[e] : 0.f;
    if (live) sr[i] = nv;
    if (q.d0) qx_store(q, i, live ? nv * nw[e] : 0.f, nv, live);
  }
}

hipError_t norm_add(hipStream_t s, const float *delta, const float *w, float *state, uint32_t n, float eps, uint32_t batch) {
  if (!batch || !n) return hipSuccess;
  if (n <= NA_T * NA_E) {
    hipLaunchKernelGGL(k_norm_add_q, dim3(batch), dim3(NA_T), 0, s, delta, w, state, n, eps, (const float *)nullptr, QXOut());
  } else {
    hipLaunchKernelGGL(k_norm_add, dim3(batch), dim3(256), 0, s, delta, w, state, n, eps);
  }
  return hipGetLastError();
}

// One row (the decode token) over many workgroups: every workgroup forms the sum of squares
// of the whole delta row itself (its loads all go out at once: raw buffer loads, zero past
// the row), then updates its own 256 elements of the state and writes their QX form. No
// workgroup waits on another, and no CU streams the row alone.
constexpr uint32_t NAW_E = 64;  // delta elements per thread: rows up to 16384
template <uint32_t E>
__global__ __launch_bounds__(256) void k_norm_add_qw(const float *d, const float *w, float *state, uint32_t n,
                                                     float eps, const float *next_w, QXOut q) {
  __shared__ float red[4];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t i = blockIdx.x * 256 + tid;
  const bool live = i < n;
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(d), 0, (int)(4 * n), 0x00020000);
  float dv[E];
#pragma unroll
  for (uint32_t e = 0; e < E; e++)
    dv[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rd, 4 * (tid + 256 * e), 0, 0));
  const float sv = live ? state[i] : 0.f, ww = live ? w[i] : 0.f, nw = live ? next_w[i] : 0.f;
  const float mine = live ? d[i] : 0.f;
  float s = 0.f;
#pragma unroll
  for (uint32_t e = 0; e < E; e++) s += dv[e] * dv[e];
  s = wave_sum(s);
  if (lane == 0) red[wv] = s;
  __syncthreads();
  s = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.f / sqrtf(s / (float)n + eps);
  const float nv = live ? sv + mine * inv * ww : 0.f;
  if (live) state[i] = nv;
  qx_store(q, i, live ? nv * nw : 0.f, nv, live);
}

hipError_t norm_add_quantize(hipStream_t s, const float *delta, const float *w, float *state, uint32_t n, float eps,
                             const float *next_w, const QXOut &q) {
  if (!n || n % 16 || !next_w) return hipErrorInvalidValue;
  if (n > 256 * NAW_E) {
    WGD_HIP(norm_add(s, delta, w, state, n, eps, 1));
    return quantize(s, state, n, next_w, q);
  }
  const dim3 grid((n + 255) / 256);
  const uint32_t per = (n + 255) / 256;  // delta elements per thread
  if (per <= 8) hipLaunchKernelGGL(k_norm_add_qw<8>, grid, dim3(256), 0, s, delta, w, state, n, eps, next_w, q);
  else if (per <= 16) hipLaunchKernelGGL(k_norm_add_qw<16>, grid, dim3(256), 0, s, delta, w, state, n, eps, next_w, q);
  else if (per <= 32) hipLaunchKernelGGL(k_norm_add_qw<32>, grid, dim3(256), 0, s, delta, w, state, n, eps, next_w, q);
  else hipLaunchKernelGGL(k_norm_add_qw<NAW_E>, grid, dim3(256), 0, s, delta, w, state, n, eps, next_w, q);
  return hipGetLastError();
}

// ------------------------------------------------------------------ RoPE
// One wavefront per (token, head). mode 0: per-head RMS with w, then half-split rotation of
// the first rot dims, tail normalised only; 1: half-split; 2: adjacent pairs.
__global__ __launch_bounds__(256) void k_rope(float *x, const float *w, uint32_t heads, uint32_t hd,
                                              uint32_t start, const int32_t *start_dev, float theta,
                                              float scale, float eps, uint32_t rot, uint32_t batch,
                                              int mode) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= heads * batch) return;
  const uint32_t t = item / heads;
  float *v = x + (uint64_t)item * hd;
  const uint32_t s0 = start_dev ? (uint32_t)*start_dev : start;
  float inv = 1.f;
  if (mode == 0) {
    float s = 0.f;
    for (uint32_t i = lane; i < hd; i += 64) s += v[i] * v[i];
    s = wave_sum(s);
    inv = 1.f / sqrtf(s / (float)hd + eps);
  }
  const double pos = (double)(s0 + t) * (double)scale;
  const uint32_t half = rot / 2;
  for (uint32_t i = lane; i < half; i += 64) {
    double angle = pos * pow((double)theta, -(double)(2 * i) / (double)rot);
    double sn, cs;
    sincos(angle, &sn, &cs);
    float c = (float)cs, sf = (float)sn;
    uint32_t ia = mode == 2 ? 2 * i : i, ib = mode == 2 ? 2 * i + 1 : i + half;
    float a = v[ia], b = v[ib];
    if (mode == 0) { a = a * w[ia] * inv; b = b * w[ib] * inv; }
    v[ia] = a * c - b * sf;
    v[ib] = a * sf + b * c;
  }
  if (mode == 0)
    for (uint32_t i = rot + lane; i < hd; i += 64) v[i] = v[i] * w[i] * inv;
}

// RoPE rotations of a batch of positions: cs[t * rot/2 + i] = (cos, sin) of
// (start + t) * scale * theta^(-2i/rot), formed in f64 as in k_rope and rounded to f32 once.
__global__ __launch_bounds__(256) void k_rope_table(float2 *cs, uint32_t half, uint32_t rot, uint32_t n,
                                                    uint32_t start, const int32_t *start_dev, float theta, float scale) {
  const uint32_t j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n * half) return;
  const uint32_t t = j / half, i = j % half;
  const uint32_t s0 = start_dev ? (uint32_t)*start_dev : start;
  const double pos = (double)(s0 + t) * (double)scale;
  const double angle = pos * pow((double)theta, -(double)(2 * i) / (double)rot);
  double sn, c;
  sincos(angle, &sn, &c);
  cs[j] = make_float2((float)c, (float)sn);
}

hipError_t rope_table(hipStream_t s, float2 *cs, uint32_t rot, uint32_t n, uint32_t start, const int32_t *start_dev,
                      float theta, float scale) {
  if (!n) return hipSuccess;
  if (!rot || rot % 2) return hipErrorInvalidValue;
  const uint32_t count = n * (rot / 2);
  hipLaunchKernelGGL(k_rope_table, dim3((count + 255) / 256), dim3(256), 0, s, cs, rot / 2, rot, n, start, start_dev,
                     theta, scale);
  return hipGetLastError();
}

// The finish of the grouped Q/K/V prompt GEMM: per (token, head) one wavefront sums the
// head's split-K partials in split order, adds the bias, applies k_rope's norm and rotation
// (rotations from rope_table, the same f64 angles) to Q and K heads, and writes Q to q and K / V straight into the
// ring slot of the token's position (k_kv_append's slot). The head is staged in LDS so any
// rotary width and pair layout can be read back.
//
// With hd 128 and a multiple of 8 head slots (by_xcd), slot s is the GEMM's 128-row tile s,
// which ran on XCD s % 8 (the tile count leads its grid; workgroups go to the XCDs
// round-robin). Workgroup w, on XCD w % 8, then takes slots s = w (mod 8), so it reads
// only partials its XCD wrote and the next GEMM's writes to the scratch take no coherence
// probes; otherwise workgroup w takes items 4w .. 4w + 3.
__global__ __launch_bounds__(256) void k_qkv_finish(QKVFinish a, uint32_t by_xcd) {
  __shared__ float buf[4][512];
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t per = a.heads + 2 * a.kvh, hd = a.hd;
  uint32_t tok, slot;
  if (by_xcd) {
    const uint32_t i = blockIdx.x / 8 * 4 + wv, per8 = per / 8;
    tok = i / per8;
    slot = blockIdx.x % 8 + 8 * (i % per8);
  } else {
    const uint32_t item = blockIdx.x * 4 + wv;
    tok = item / per;
    slot = item % per;
  }
  if (tok >= a.batch) return;
  const int kind = slot < a.heads ? 0 : slot < a.heads + a.kvh ? 1 : 2;
  const uint32_t h = kind == 0 ? slot : kind == 1 ? slot - a.heads : slot - a.heads - a.kvh;
  const float *bias = kind == 0 ? a.bq : kind == 1 ? a.bk : a.bv;
  const uint64_t n = (uint64_t)a.rows_total * a.batch, base = (uint64_t)tok * a.rows_total + (uint64_t)slot * hd;
  float *v = buf[wv];
  const __amdgpu_buffer_rsrc_t rp = split_rsrc(a.part, a.splits, n);
  const float xinv = deferred_inv(a.xnorm, tok);
  for (uint32_t d = lane; d < hd; d += 64) {
    float acc = split_sum<MAX_SPLITS>(rp, a.splits, (uint32_t)(4 * n), (uint32_t)(4 * (base + d)));
    if (a.xnorm.sq) acc *= xinv;
    v[d] = bias ? acc + bias[h * hd + d] : acc;
  }
  __builtin_amdgcn_wave_barrier();
  const uint32_t s0 = a.start_dev ? (uint32_t)*a.start_dev : a.start;
  const uint64_t ring = (uint64_t)((s0 + tok) % a.capacity) * a.kvh * hd + (uint64_t)h * hd;
  // Q rows go to q (f32); K/V rows to the ring (f32, or f16 rounded to nearest even)
  void *dst = kind == 0 ? (void *)(a.q + ((uint64_t)tok * a.heads + h) * hd) : kind == 1 ? a.kc : a.vc;
  const uint64_t d0 = kind == 0 ? 0 : ring;
  const bool f16 = kind != 0 && a.kv16;
  if (kind == 2) {
    for (uint32_t d = lane; d < hd; d += 64) kv_put(dst, d0 + d, v[d], f16);
    return;
  }
  const float *w = kind == 0 ? a.qn : a.kn;
  float inv = 1.f;
  if (a.mode == 0) {
    float ss = 0.f;
    for (uint32_t d = lane; d < hd; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    inv = 1.f / sqrtf(ss / (float)hd + a.eps);
  }
  const uint32_t half = a.rot / 2;
  for (uint32_t i = lane; i < half; i += 64) {
    const float2 t = a.cs[(uint64_t)tok * half + i];
    const float c = t.x, sf = t.y;
    const uint32_t ia = a.mode == 2 ? 2 * i : i, ib = a.mode == 2 ? 2 * i + 1 : i + half;
    float x0 = v[ia], x1 = v[ib];
    if (a.mode == 0) { x0 = x0 * w[ia] * inv; x1 = x1 * w[ib] * inv; }
    kv_put(dst, d0 + ia, x0 * c - x1 * sf, f16);
    kv_put(dst, d0 + ib, x0 * sf + x1 * c, f16);
  }
  for (uint32_t d = a.rot + lane; d < hd; d += 64) kv_put(dst, d0 + d, a.mode == 0 ? v[d] * w[d] * inv : v[d], f16);
}

hipError_t qkv_finish(hipStream_t s, const QKVFinish &a) {
  if (!a.batch) return hipSuccess;
  if (a.hd > 512 || a.rot > a.hd || a.rot % 2 || !a.capacity || !a.cs || (a.mode == 0 && (!a.qn || !a.kn)) ||
      !a.splits || a.splits > MAX_SPLITS || (uint64_t)a.splits * a.rows_total * a.batch * 4 >= (1ull << 31))
    return hipErrorInvalidValue;
  const uint32_t per = a.heads + 2 * a.kvh, items = a.batch * per;
  const uint32_t by_xcd = a.hd == 128 && per % 8 == 0 ? 1u : 0u;
  const uint32_t groups = by_xcd ? 8 * ((a.batch * (per / 8) + 3) / 4) : (items + 3) / 4;
  hipLaunchKernelGGL(k_qkv_finish, dim3(groups), dim3(256), 0, s, a, by_xcd);
  return hipGetLastError();
}

hipError_t rope(hipStream_t s, float *x, const float *w, uint32_t heads, uint32_t hd, uint32_t start,
                const int32_t *start_dev, float theta, float scale, float eps, uint32_t rotary_dim,
                uint32_t batch, int mode) {
  if (!batch || !heads) return hipSuccess;
  uint32_t rot = rotary_dim ? rotary_dim : hd;
  uint32_t items = heads * batch;
  hipLaunchKernelGGL(k_rope, dim3((items + 3) / 4), dim3(256), 0, s, x, w, heads, hd, start, start_dev, theta,
                     scale, eps, rot, batch, mode);
  return hipGetLastError();
}

// ------------------------------------------------------------------ elementwise
__global__ void k_add(const float *d, float *state, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) state[i] += d[i];
}
__global__ void k_glu(const float *g, const float *u, float *y, uint32_t n, int act) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float x = g[i];
    y[i] = glu_act(x, act) * u[i];
  }
}
__global__ void k_bias(float *y, const float *b, uint32_t n, uint32_t width) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) y[i] += b[i % width];
}
__global__ void k_activate(float *x, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) { float v = x[i]; x[i] = v / (1.f + expf(-v)); }
}

static dim3 grid_for(uint32_t n) { uint32_t g = (n + 255) / 256; if (g > 4096) g = 4096; if (!g) g = 1; return dim3(g); }

hipError_t add(hipStream_t s, const float *delta, float *state, uint32_t n) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_add, grid_for(n), dim3(256), 0, s, delta, state, n);
  return hipGetLastError();
}
hipError_t glu(hipStream_t s, const float *gate, const float *up, float *y, uint32_t n, int act) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_glu, grid_for(n), dim3(256), 0, s, gate, up, y, n, act);
  return hipGetLastError();
}

// Eight consecutive elements of one token per thread.
__global__ __launch_bounds__(256) void k_glu_split(const float *g, const float *u, float *y, uint16_t *xs,
                                                   uint32_t cols, uint32_t count, int act) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const uint32_t c8 = cols / 8, tok = i / c8, k = (i % c8) * 8;
  const uint64_t o = (uint64_t)tok * cols + k;
  float v[8];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const float4 gv = *(const float4 *)(g + o + 4 * h), uv = *(const float4 *)(u + o + 4 * h);
    const float gg[4] = {gv.x, gv.y, gv.z, gv.w}, uu[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float x = gg[e];
      v[4 * h + e] = glu_act(x, act) * uu[e];
    }
  }
  const float4 a = make_float4(v[0], v[1], v[2], v[3]), b = make_float4(v[4], v[5], v[6], v[7]);
  *(float4 *)(y + o) = a;
  *(float4 *)(y + o + 4) = b;
  split_store8(xs, cols, tok, k, a, b);
}

hipError_t glu_split(hipStream_t s, const float *gate, const float *up, float *y, uint16_t *xs, uint32_t cols,
                     uint32_t batch, int act) {
  if (!batch) return hipSuccess;
  if (cols % SPLIT_K || ((uintptr_t)gate | (uintptr_t)up | (uintptr_t)y) % 16) return hipErrorInvalidValue;
  const uint32_t count = batch * (cols / 8);
  hipLaunchKernelGGL(k_glu_split, dim3((count + 255) / 256), dim3(256), 0, s, gate, up, y, xs, cols, count, act);
  return hipGetLastError();
}
hipError_t bias_add(hipStream_t s, float *y, const float *b, uint32_t n, uint32_t width) {
  if (!n) return hipSuccess;
  if (!width) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_bias, grid_for(n), dim3(256), 0, s, y, b, n, width);
  return hipGetLastError();
}
hipError_t activate(hipStream_t s, float *x, uint32_t n) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_activate, grid_for(n), dim3(256), 0, s, x, n);
  return hipGetLastError();
}

// ------------------------------------------------------------------ KV ring append
__global__ void k_kv_append(const float *k, const float *v, void *kc, void *vc, uint32_t row, uint32_t n,
                            uint32_t start, const int32_t *start_dev, uint32_t capacity, bool f16) {
  const uint32_t s0 = start_dev ? (uint32_t)*start_dev : start;
  const uint64_t total = (uint64_t)n * row;
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
    uint32_t t = (uint32_t)(i / row), e = (uint32_t)(i % row);
    uint64_t slot = (uint64_t)((s0 + t) % capacity) * row + e;
    kv_put(kc, slot, k[i], f16);
    kv_put(vc, slot, v[i], f16);
  }
}

hipError_t kv_append(hipStream_t s, const float *k, const float *v, void *kc, void *vc, uint32_t row_floats,
                     uint32_t n, uint32_t start, const int32_t *start_dev, uint32_t capacity, bool kv16) {
  if (!n) return hipSuccess;
  if (!capacity) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_kv_append, grid_for(n * row_floats), dim3(256), 0, s, k, v, kc, vc, row_floats, n, start,
                     start_dev, capacity, kv16);
  return hipGetLastError();
}

__global__ void k_to_f16(const float *src, _Float16 *dst, uint64_t n) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = (_Float16)src[i];
}

hipError_t to_f16(hipStream_t s, const float *src, _Float16 *dst, uint64_t n) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_to_f16, grid_for(n < (1u << 30) ? (uint32_t)n : (1u << 30)), dim3(256), 0, s, src, dst, n);
  return hipGetLastError();
}

// ------------------------------------------------------------------ argmax
__global__ __launch_bounds__(256) void k_argmax_partial(const float *x, uint32_t n, uint64_t *part) {
  __shared__ uint64_t red[4];
  uint64_t k = 0;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) k = key_max(k, arg_key(x[i], i));
  k = wave_max_key(k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = key_max(key_max(red[0], red[1]), key_max(red[2], red[3]));
}
__global__ __launch_bounds__(256) void k_argmax_final(const uint64_t *part, uint32_t np, int32_t *out) {
  __shared__ uint64_t red[4];
  uint64_t k = 0;
  for (uint32_t i = threadIdx.x; i < np; i += 256) k = key_max(k, part[i]);
  k = wave_max_key(k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t m = key_max(key_max(red[0], red[1]), key_max(red[2], red[3]));
    *out = m ? (int32_t)(0xFFFFFFFFu - (uint32_t)m) : -1;
  }
}

// Scratch for the partial keys lives right after the int32 result (out must point into
// a buffer of at least 8 + 8 * 256 bytes, 8-byte aligned past out).
hipError_t argmax(hipStream_t s, const float *logits, uint32_t n, int32_t *out) {
  uint32_t blocks = (n + 4095) / 4096; if (blocks > 256) blocks = 256; if (!blocks) blocks = 1;
  uint64_t *part = (uint64_t *)((uint8_t *)out + 8);
  hipLaunchKernelGGL(k_argmax_partial, dim3(blocks), dim3(256), 0, s, logits, n, part);
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, part, blocks, out);
  return hipGetLastError();
}

}  // namespace wgd
