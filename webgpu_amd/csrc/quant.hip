// quant.hip — GGUF block decode, embedding gather and the decode dequant-matvec (gfx950).
//
// Exact decode (deq_elem) restates decodeWeight, src/core/quant.ts:6-29: every product is
// exact in f32, so each weight equals RN_f32 of its exact value, bit-identical to the
// reference. The matvec replaces matmulShader (src/core/shaders.ts:39-54): instead of one
// 64-lane workgroup per row re-decoding every element with byte loads, a wavefront owns a
// row and each lane owns whole 64-weight units of a super-block, read with 16-byte loads.
// The activation row is staged once per workgroup in LDS together with its 32- or
// 16-element partial sums, so the affine Q4_K minimum and the Q6_K/Q8_0 offsets are
// applied once per sub-block: sum_j (d*sc*q_j - dmin*m) x_j = d*sc*sum_j q_j x_j - dmin*m*sum_j x_j.
#include "internal.h"
#include "decode.h"
#include "model.h"

namespace wgd {

__global__ void k_dequant(int type, const uint8_t *w, float *out, uint64_t count) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
    out[i] = deq_elem(type, w, i);
}

hipError_t dequant(hipStream_t s, int type, const uint8_t *w, float *out, uint64_t count) {
  if (!count) return hipSuccess;
  uint64_t blocks = (count + 255) / 256; if (blocks > 65535 * 16) blocks = 65535 * 16;
  hipLaunchKernelGGL(k_dequant, dim3((uint32_t)blocks), dim3(256), 0, s, type, w, out, count);
  return hipGetLastError();
}

// Embedding row gather: out[b][i] = f32(deq(table)[ids[b]][i] * scale), product in f64 as
// the reference's JS computes decodeWeight(...) * Math.sqrt(hidden) (engine.ts:143).
__global__ void k_embed(int type, const uint8_t *table, const int32_t *ids, float *out,
                        uint32_t hidden, uint64_t rb, double scale) {
  uint32_t b = blockIdx.y;
  const uint8_t *row = table + (uint64_t)ids[b] * rb;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
    float v = deq_elem(type, row, i);
    out[(uint64_t)b * hidden + i] = scale == 1.0 ? v : (float)((double)v * scale);
  }
}

hipError_t embed(hipStream_t s, int type, const uint8_t *table, const int32_t *ids, float *out,
                 uint32_t hidden, uint32_t n, double scale) {
  if (!n) return hipSuccess;
  uint32_t gx = (hidden + 255) / 256; if (gx > 64) gx = 64;
  hipLaunchKernelGGL(k_embed, dim3(gx, n), dim3(256), 0, s, type, table, ids, out, hidden, row_bytes(type, hidden), scale);
  return hipGetLastError();
}

// Gather from a planar Q6_K / Q8_0 table: element i of `row`, decoded exactly as deq_elem.
__device__ __forceinline__ float deq_planar(int type, const uint8_t *w, uint64_t nbt, uint32_t bpr, uint32_t row, uint32_t i) {
  uint64_t bi = (uint64_t)row * bpr + i / block_size_dev(type);
  if (type == Q6_K) {
    Q6Planes p = q6_planes(nbt);
    uint32_t j = i % 256, seg = j / 128, qtr = (j % 128) / 32, ln = j % 32;
    uint32_t lo = (w[p.ql + bi * 128 + seg * 64 + (qtr % 2) * 32 + ln] >> ((qtr / 2) * 4)) & 15u;
    uint32_t hi = (w[p.qh + bi * 64 + seg * 32 + ln] >> (qtr * 2)) & 3u;
    float sc = (float)(int8_t)w[p.sc + bi * 16 + seg * 8 + qtr * 2 + ln / 16];
    return half_bits(w[p.d + bi * 2] | ((uint32_t)w[p.d + bi * 2 + 1] << 8)) * sc * (float)((int)(lo | (hi << 4)) - 32);
  }
  Q8Planes p = q8_planes(nbt);
  return half_bits(w[p.d + bi * 2] | ((uint32_t)w[p.d + bi * 2 + 1] << 8)) * (float)(int8_t)w[p.qs + bi * 32 + i % 32];
}

__global__ void k_embed_planar(int type, const uint8_t *table, uint64_t nbt, uint32_t bpr, const int32_t *ids, float *out,
                               uint32_t hidden, double scale) {
  uint32_t b = blockIdx.y, row = (uint32_t)ids[b];
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
    float v = deq_planar(type, table, nbt, bpr, row, i);
    out[(uint64_t)b * hidden + i] = scale == 1.0 ? v : (float)((double)v * scale);
  }
}

hipError_t embed_matrix(hipStream_t s, const Matrix &t, const int32_t *ids, float *out, uint32_t n, double scale) {
  if (t.layout == LAYOUT_GGUF) return embed(s, t.type, t.data, ids, out, t.cols, n, scale);
  if (!n) return hipSuccess;
  uint32_t gx = (t.cols + 255) / 256; if (gx > 64) gx = 64;
  uint32_t bpr = t.cols / block_size(t.type);
  hipLaunchKernelGGL(k_embed_planar, dim3(gx, n), dim3(256), 0, s, t.type, t.data, (uint64_t)bpr * t.rows, bpr, ids, out,
                     t.cols, scale);
  return hipGetLastError();
}

// ------------------------------------------------------------------ planar repack

bool has_planar(int type) { return type == Q6_K || type == Q8_0; }

__global__ void k_repack_q6(const uint8_t *src, uint8_t *dst, uint64_t nb) {
  Q6Planes p = q6_planes(nb);
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < nb * 210; i += (uint64_t)gridDim.x * blockDim.x) {
    uint64_t blk = i / 210; uint32_t o = i % 210; uint8_t v = src[i];
    if (o < 128) dst[p.ql + blk * 128 + o] = v;
    else if (o < 192) dst[p.qh + blk * 64 + (o - 128)] = v;
    else if (o < 208) dst[p.sc + blk * 16 + (o - 192)] = v;
    else dst[p.d + blk * 2 + (o - 208)] = v;
  }
}
__global__ void k_repack_q8(const uint8_t *src, uint8_t *dst, uint64_t nb) {
  Q8Planes p = q8_planes(nb);
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < nb * 34; i += (uint64_t)gridDim.x * blockDim.x) {
    uint64_t blk = i / 34; uint32_t o = i % 34; uint8_t v = src[i];
    if (o < 2) dst[p.d + blk * 2 + o] = v; else dst[p.qs + blk * 32 + (o - 2)] = v;
  }
}

hipError_t repack_planar(hipStream_t s, int type, const uint8_t *src, uint8_t *dst, uint64_t blocks) {
  if (!blocks) return hipSuccess;
  uint64_t bytes = blocks * block_bytes(type), grid = (bytes + 255) / 256; if (grid > 65535 * 8) grid = 65535 * 8;
  if (type == Q6_K) hipLaunchKernelGGL(k_repack_q6, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, blocks);
  else if (type == Q8_0) hipLaunchKernelGGL(k_repack_q8, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, blocks);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// ------------------------------------------------------------------ generic matmul
// Any type, any batch; the reference algorithm with a lane-strided f32 sum per row and a
// wave reduction. Used for the known-answer checks, F32/F16 tensors and fallbacks.
__global__ __launch_bounds__(256) void k_matmul_generic(int type, const uint8_t *w, uint64_t rb,
    const float *x, float *y, uint32_t cols, uint32_t rows, uint32_t stride, uint32_t row_base,
    uint32_t input_offset, uint32_t batch) {
  uint32_t lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint8_t *wr = w + (uint64_t)row * rb;
  for (uint32_t b0 = blockIdx.y * 4; b0 < batch; b0 += gridDim.y * 4) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    uint32_t nb = batch - b0 < 4 ? batch - b0 : 4;
    for (uint32_t c = lane; c < cols; c += 64) {
      float wv = deq_elem(type, wr, c);
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (j < (int)nb) acc[j] += wv * x[(uint64_t)(b0 + j + input_offset) * cols + c];
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float r = wave_sum(acc[j]);
      if (lane == 0 && j < (int)nb) y[(uint64_t)(b0 + j) * stride + row_base + row] = r;
    }
  }
}

hipError_t matmul_generic(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                          uint32_t row_base, uint32_t input_offset, uint32_t batch) {
  if (!w.rows || !batch) return hipSuccess;
  if (w.layout != LAYOUT_GGUF) return hipErrorInvalidValue;
  uint32_t gy = (batch + 3) / 4; if (gy > 32) gy = 32;
  hipLaunchKernelGGL(k_matmul_generic, dim3((w.rows + 3) / 4, gy), dim3(256), 0, s, w.type, w.data,
                     row_bytes(w.type, w.cols), x, y, w.cols, w.rows, stride, row_base, input_offset, batch);
  return hipGetLastError();
}

// ------------------------------------------------------------------ fast matvec

// Per-type unit definitions. A unit is the work of one lane for one row: UNIT weights
// read with aligned 16-byte loads, UNIT activations held in registers (reused across the
// rows a wavefront visits), plus the partial sums SEG-wide of those activations.
struct Q4K {
  static constexpr int UNIT = 64, SEG = 32, NSUM = 2;  // unit = (block, 32-byte quant group)
  static __device__ __forceinline__ uint32_t units(uint32_t cols) { return cols / 64; }
  // x index of element e (0..63) of unit u: block b = u/4, group g = u%4 -> 64 consecutive.
  static __device__ __forceinline__ uint32_t xbase(uint32_t u) { return u * 64; }
  static __device__ __forceinline__ void load_x(const float *xs, const float *ss, uint32_t u, float *xv, float *sv) {
    const float4 *p = (const float4 *)(xs + u * 64);
#pragma unroll
    for (int i = 0; i < 16; i++) { float4 t = p[i]; xv[4 * i] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w; }
    sv[0] = ss[2 * u]; sv[1] = ss[2 * u + 1];
  }
  struct Raw { uint4 h, a, b; };
  static __device__ __forceinline__ Raw load(const uint8_t *w, uint64_t rb, uint32_t nb_unused, uint32_t row, uint32_t u) {
    const uint8_t *blk = w + (uint64_t)row * rb + (uint64_t)(u >> 2) * 144;
    uint32_t g = u & 3;
    Raw r;
    r.h = *(const uint4 *)blk;
    r.a = *(const uint4 *)(blk + 16 + 32 * g);
    r.b = *(const uint4 *)(blk + 32 + 32 * g);
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw &r, uint32_t u, const float *xv, const float *sv) {
    uint32_t g = u & 3, sh = 16 * (g & 1);
    uint32_t A = r.h.y, B = r.h.z, C = r.h.w;
    uint32_t sc0, sc1, m0, m1;
    if (g < 2) {  // sub-blocks 2g, 2g+1 < 4: six bits of scale bytes 0..3 / 4..7
      sc0 = (A >> sh) & 63u; sc1 = (A >> (sh + 8)) & 63u;
      m0 = (B >> sh) & 63u; m1 = (B >> (sh + 8)) & 63u;
    } else {      // sub-blocks 4..7: low nibbles in bytes 8..11, top two bits in bytes 0..7
      sc0 = ((C >> sh) & 15u) | (((A >> sh) >> 6 & 3u) << 4);
      sc1 = ((C >> (sh + 8)) & 15u) | (((A >> (sh + 8)) >> 6 & 3u) << 4);
      m0 = ((C >> sh) >> 4 & 15u) | (((B >> sh) >> 6 & 3u) << 4);
      m1 = ((C >> (sh + 8)) >> 4 & 15u) | (((B >> (sh + 8)) >> 6 & 3u) << 4);
    }
    uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        a0 += (float)((lo >> (8 * j)) & 0xFFu) * xv[4 * k + j];
        a1 += (float)((hi >> (8 * j)) & 0xFFu) * xv[32 + 4 * k + j];
      }
    }
    float d = half_bits(r.h.x & 0xFFFFu), dm = half_bits(r.h.x >> 16);
    return d * ((float)sc0 * a0 + (float)sc1 * a1) - dm * ((float)m0 * sv[0] + (float)m1 * sv[1]);
  }
};

// Q6_K in the planar layout. Unit = (block, 128-element half, 16-lane half): 64 weights
// from two 16-byte low-nibble loads, one 16-byte high-bit load and 4 signed scales.
struct Q6K {
  static constexpr int UNIT = 64, SEG = 16, NSUM = 4;
  static __device__ __forceinline__ uint32_t units(uint32_t cols) { return cols / 64; }
  // elements of unit u (b = u/4, seg = (u/2)&1, h = u&1): for quarter t, 16 consecutive at
  // b*256 + seg*128 + t*32 + 16h.
  static __device__ __forceinline__ void load_x(const float *xs, const float *ss, uint32_t u, float *xv, float *sv) {
    uint32_t b = u >> 2, seg = (u >> 1) & 1, h = u & 1;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      uint32_t base = b * 256 + seg * 128 + t * 32 + 16 * h;
      const float4 *p = (const float4 *)(xs + base);
#pragma unroll
      for (int i = 0; i < 4; i++) { float4 v = p[i]; xv[16 * t + 4 * i] = v.x; xv[16 * t + 4 * i + 1] = v.y; xv[16 * t + 4 * i + 2] = v.z; xv[16 * t + 4 * i + 3] = v.w; }
      sv[t] = ss[base / 16];
    }
  }
  struct Raw { uint4 a, b, h; uint2 s; uint32_t d; };
  static __device__ __forceinline__ Raw load_planar(const uint8_t *w, uint64_t nbt, uint32_t bpr, uint32_t row, uint32_t u) {
    Q6Planes p = q6_planes(nbt);
    uint64_t bi = (uint64_t)row * bpr + (u >> 2);
    uint32_t seg = (u >> 1) & 1, h = u & 1;
    Raw r;
    const uint8_t *ql = w + p.ql + bi * 128 + seg * 64 + 16 * h;
    r.a = *(const uint4 *)ql;
    r.b = *(const uint4 *)(ql + 32);
    r.h = *(const uint4 *)(w + p.qh + bi * 64 + seg * 32 + 16 * h);
    r.s = *(const uint2 *)(w + p.sc + bi * 16 + seg * 8);
    r.d = *(const uint16_t *)(w + p.d + bi * 2);
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw &r, uint32_t u, const float *xv, const float *sv) {
    uint32_t h = u & 1;
    uint32_t qa[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, qb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    uint32_t qh[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      // scale byte index seg*8 + t*2 + h within the 8 loaded bytes
      uint32_t sw = (t < 2) ? r.s.x : r.s.y;
      float sc = (float)(int8_t)((sw >> (8 * ((2 * t + h) & 3))) & 0xFFu);
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t src = (t & 1) ? qb[k] : qa[k];
        uint32_t lo = (t & 2) ? ((src >> 4) & 0x0F0F0F0Fu) : (src & 0x0F0F0F0Fu);
        uint32_t q = lo | (((qh[k] >> (2 * t)) & 0x03030303u) << 4);
#pragma unroll
        for (int j = 0; j < 4; j++) a += (float)((q >> (8 * j)) & 0xFFu) * xv[16 * t + 4 * k + j];
      }
      acc += sc * (a - 32.f * sv[t]);
    }
    return half_bits(r.d) * acc;
  }
};

// Q8_0 in the planar layout. Unit = one 32-element block (2 x 16-byte loads + scale).
struct Q80 {
  static constexpr int UNIT = 32, SEG = 32, NSUM = 1;
  static __device__ __forceinline__ uint32_t units(uint32_t cols) { return cols / 32; }
  static __device__ __forceinline__ void load_x(const float *xs, const float *ss, uint32_t u, float *xv, float *sv) {
    const float4 *p = (const float4 *)(xs + u * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) { float4 t = p[i]; xv[4 * i] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w; }
    sv[0] = ss[u];
  }
  struct Raw { uint4 a, b; uint32_t d; };
  static __device__ __forceinline__ Raw load_planar(const uint8_t *w, uint64_t nbt, uint32_t bpr, uint32_t row, uint32_t u) {
    Q8Planes p = q8_planes(nbt);
    uint64_t bi = (uint64_t)row * bpr + u;
    Raw r;
    r.a = *(const uint4 *)(w + p.qs + bi * 32);
    r.b = *(const uint4 *)(w + p.qs + bi * 32 + 16);
    r.d = *(const uint16_t *)(w + p.d + bi * 2);
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw &r, uint32_t u, const float *xv, const float *sv) {
    uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      uint32_t v = q[k] ^ 0x80808080u;  // int8 + 128 as unsigned bytes
#pragma unroll
      for (int j = 0; j < 4; j++) a += (float)((v >> (8 * j)) & 0xFFu) * xv[4 * k + j];
    }
    return half_bits(r.d) * (a - 128.f * sv[0]);
  }
};

template <class T> struct Loader;
template <> struct Loader<Q4K> {
  static __device__ __forceinline__ Q4K::Raw load(const uint8_t *w, uint64_t rb, uint64_t, uint32_t, uint32_t row, uint32_t u) { return Q4K::load(w, rb, 0, row, u); }
};
template <> struct Loader<Q6K> {
  static __device__ __forceinline__ Q6K::Raw load(const uint8_t *w, uint64_t, uint64_t nbt, uint32_t bpr, uint32_t row, uint32_t u) { return Q6K::load_planar(w, nbt, bpr, row, u); }
};
template <> struct Loader<Q80> {
  static __device__ __forceinline__ Q80::Raw load(const uint8_t *w, uint64_t, uint64_t nbt, uint32_t bpr, uint32_t row, uint32_t u) { return Q80::load_planar(w, nbt, bpr, row, u); }
};

enum Epilogue : int { EPI_STORE = 0, EPI_ADD = 1, EPI_GLU_SILU = 2, EPI_GLU_GELU = 3 };

struct MatvecArgs {
  const uint8_t *w0, *w1;   // w1: the "up" matrix of a gated pair
  uint64_t rb, nbt;         // GGUF row bytes / total blocks (planar)
  uint32_t bpr;             // blocks per row
  const float *x; float *y;
  uint32_t cols, rows, row_base;
  const float *norm_w; float eps;
  int epi;
};

__device__ __forceinline__ float gelu_tanh(float g) {
  return 0.5f * g * (1.f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g)));
}

// One workgroup = 4 wavefronts. The activation row (optionally RMS-normalised) and its
// SEG-wide sums are staged in LDS once; each wavefront then walks R rows at a time, each
// lane holding the activations of its units in registers across those rows.
template <class T, int R>
__global__ __launch_bounds__(256) void k_matvec(MatvecArgs a) {
  extern __shared__ float lds[];
  float *xs = lds, *ss = lds + a.cols;
  __shared__ float red[4];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float inv = 1.f;
  if (a.norm_w) {
    float s = 0.f;
    for (uint32_t i = tid; i < a.cols; i += 256) { float v = a.x[i]; s += v * v; }
    s = wave_sum(s);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    s = red[0] + red[1] + red[2] + red[3];
    inv = 1.f / sqrtf(s / (float)a.cols + a.eps);
  }
  for (uint32_t i = tid * 4; i < a.cols; i += 1024) {
    float4 v = *(const float4 *)(a.x + i);
    if (a.norm_w) {
      float4 g = *(const float4 *)(a.norm_w + i);
      v.x = v.x * inv * g.x; v.y = v.y * inv * g.y; v.z = v.z * inv * g.z; v.w = v.w * inv * g.w;
    }
    *(float4 *)(xs + i) = v;
  }
  __syncthreads();
  for (uint32_t sgi = tid; sgi < a.cols / T::SEG; sgi += 256) {
    float s = 0.f;
#pragma unroll 8
    for (int j = 0; j < T::SEG; j++) s += xs[sgi * T::SEG + j];
    ss[sgi] = s;
  }
  __syncthreads();

  const uint32_t U = T::units(a.cols);
  // Lanes per row: all 64 when a row has >= 64 units, else the power-of-two segment
  // covering U so several rows share one wavefront pass.
  uint32_t width = 64;
  while (width > 1 && (width >> 1) >= U) width >>= 1;
  const uint32_t per_pass = 64 / width, seg_id = lane / width, ul = lane % width;
  const uint32_t rows_per_wg = 4 * R * per_pass;
  const uint32_t groups = (a.rows + rows_per_wg - 1) / rows_per_wg;
  for (uint32_t grp = blockIdx.x; grp < groups; grp += gridDim.x) {
    const uint32_t row0 = grp * rows_per_wg + (wv * R) * per_pass + seg_id;
    float acc0[R], acc1[R];
#pragma unroll
    for (int r = 0; r < R; r++) { acc0[r] = 0.f; acc1[r] = 0.f; }
    for (uint32_t u = ul; u < U; u += width) {
      float xv[T::UNIT], sv[T::NSUM];
      T::load_x(xs, ss, u, xv, sv);
      typename T::Raw raw0[R], raw1[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        uint32_t row = row0 + r * per_pass;
        if (row < a.rows) {
          raw0[r] = Loader<T>::load(a.w0, a.rb, a.nbt, a.bpr, row, u);
          if (a.epi >= EPI_GLU_SILU) raw1[r] = Loader<T>::load(a.w1, a.rb, a.nbt, a.bpr, row, u);
        }
      }
#pragma unroll
      for (int r = 0; r < R; r++) {
        uint32_t row = row0 + r * per_pass;
        if (row < a.rows) {
          acc0[r] += T::dot(raw0[r], u, xv, sv);
          if (a.epi >= EPI_GLU_SILU) acc1[r] += T::dot(raw1[r], u, xv, sv);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint32_t row = row0 + r * per_pass;
      float g = segment_sum(acc0[r], width);
      float up = a.epi >= EPI_GLU_SILU ? segment_sum(acc1[r], width) : 0.f;
      if (ul == 0 && row < a.rows) {
        float* dst = a.y + a.row_base + row;
        if (a.epi == EPI_STORE) *dst = g;
        else if (a.epi == EPI_ADD) *dst += g;
        else if (a.epi == EPI_GLU_SILU) *dst = g / (1.f + expf(-g)) * up;
        else *dst = gelu_tanh(g) * up;
      }
    }
  }
}

static int g_cus = 0;
int device_cu_count() {
  if (!g_cus) {
    int dev = 0; hipGetDevice(&dev);
    hipDeviceProp_t p; if (hipGetDeviceProperties(&p, dev) == hipSuccess) g_cus = p.multiProcessorCount;
    if (g_cus <= 0) g_cus = 256;
  }
  return g_cus;
}

static size_t lds_limit() {
  static size_t lim = 0;
  if (!lim) {
    int dev = 0; hipGetDevice(&dev);
    hipDeviceProp_t p;
    lim = hipGetDeviceProperties(&p, dev) == hipSuccess ? p.sharedMemPerBlock : 65536;
    if (lim < 65536) lim = 65536;
  }
  return lim;
}

static bool fast_type(const Matrix &w) {
  if (w.type == Q4_K) return w.layout == LAYOUT_GGUF && w.cols % 256 == 0;
  if (w.type == Q6_K) return w.layout == LAYOUT_PLANAR && w.cols % 256 == 0;
  if (w.type == Q8_0) return w.layout == LAYOUT_PLANAR && w.cols % 32 == 0;
  return false;
}

bool fast_matvec_ok(const Matrix &w) {
  if (!fast_type(w)) return false;
  size_t need = (size_t)w.cols * 4 + (size_t)(w.cols / 16) * 4 + 64;
  return need <= lds_limit();
}

template <class T, int R>
static hipError_t launch_mv(hipStream_t s, const MatvecArgs &a) {
  uint32_t U = a.cols / T::UNIT;
  uint32_t width = 64;
  while (width > 1 && (width >> 1) >= U) width >>= 1;
  uint32_t rows_per_wg = 4 * R * (64 / width);
  uint32_t groups = (a.rows + rows_per_wg - 1) / rows_per_wg;
  uint32_t cap = (uint32_t)device_cu_count() * 8;
  uint32_t grid = groups < cap ? groups : cap;
  size_t lds = (size_t)a.cols * 4 + (size_t)(a.cols / T::SEG) * 4;
  if (lds > 65536) (void)hipFuncSetAttribute((const void *)k_matvec<T, R>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL((k_matvec<T, R>), dim3(grid), dim3(256), lds, s, a);
  return hipGetLastError();
}

template <class T>
static hipError_t launch_mv_rows(hipStream_t s, const MatvecArgs &a) {
  // Few rows per wavefront when the matrix is short, so the grid still fills the chip.
  uint32_t cus = (uint32_t)device_cu_count();
  if (a.rows >= cus * 4 * 4 * 2) return launch_mv<T, 4>(s, a);
  if (a.rows >= cus * 4 * 2 * 2) return launch_mv<T, 2>(s, a);
  return launch_mv<T, 1>(s, a);
}

static hipError_t launch_fast(hipStream_t s, const Matrix &w, const Matrix *w1, const float *x, float *y,
                              uint32_t row_base, NormIn norm, int epi) {
  MatvecArgs a;
  a.w0 = w.data; a.w1 = w1 ? w1->data : nullptr;
  a.rb = row_bytes(w.type, w.cols);
  a.bpr = w.cols / block_size(w.type);
  a.nbt = (uint64_t)a.bpr * w.rows;
  a.x = x; a.y = y; a.cols = w.cols; a.rows = w.rows; a.row_base = row_base;
  a.norm_w = norm.w; a.eps = norm.eps; a.epi = epi;
  switch (w.type) {
    case Q4_K: return launch_mv_rows<Q4K>(s, a);
    case Q6_K: return launch_mv_rows<Q6K>(s, a);
    case Q8_0: return launch_mv_rows<Q80>(s, a);
  }
  return hipErrorInvalidValue;
}

hipError_t matmul(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                  uint32_t row_base, uint32_t input_offset, uint32_t batch, NormIn norm) {
  if (!w.rows || !batch) return hipSuccess;
  if (batch == 1 && fast_matvec_ok(w))
    return launch_fast(s, w, nullptr, x + (uint64_t)input_offset * w.cols, y, row_base, norm, EPI_STORE);
  if (norm.w) return hipErrorInvalidValue;  // fused norm exists only on the fast path
  if ((batch > 4 || w.layout != LAYOUT_GGUF) && w.cols % 64 == 0)
    return gemm(s, w, x, y, stride, row_base, input_offset, batch);
  return matmul_generic(s, w, x, y, stride, row_base, input_offset, batch);
}

hipError_t matmul_add(hipStream_t s, const Matrix &w, const float *x, float *y) {
  return launch_fast(s, w, nullptr, x, y, 0, NormIn{}, EPI_ADD);
}

hipError_t matvec_glu(hipStream_t s, const Matrix &wg, const Matrix &wu, const float *x, float *y,
                      int act, NormIn norm) {
  if (wg.type != wu.type || wg.layout != wu.layout || wg.cols != wu.cols || wg.rows != wu.rows || !fast_matvec_ok(wg))
    return hipErrorInvalidValue;
  return launch_fast(s, wg, &wu, x, y, 0, norm, act ? EPI_GLU_GELU : EPI_GLU_SILU);
}

}  // namespace wgd
