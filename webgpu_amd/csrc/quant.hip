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
#include <mutex>
#include <unordered_set>

#include "internal.h"
#include "decode.h"
#include "model.h"
#include "matvec.h"
#include "attention.h"

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

// Gather from a planar table: element i of `row`, decoded exactly as deq_elem.
__device__ __forceinline__ float deq_planar(int type, const uint8_t *w, uint64_t nbp, uint32_t bpr, uint32_t cols,
                                            uint32_t row, uint32_t i) {
  if (type == Q4_K) {
    const uint8_t *h = w + q4_planes(nbp).hdr + tiled(row, i / 256, bpr) * 16;
    const uint32_t j = i % 256, s = j / 32;
    uint32_t sc, mn;
    if (s < 4) { sc = h[4 + s] & 63u; mn = h[8 + s] & 63u; }
    else { sc = (h[8 + s] & 15u) | ((h[s] >> 6) << 4); mn = (h[8 + s] >> 4) | ((h[4 + s] >> 6) << 4); }
    const uint32_t q = q4_quant(w, row, cols / 32, i);
    return half_bits(h[0] | ((uint32_t)h[1] << 8)) * (float)(sc * q) - half_bits(h[2] | ((uint32_t)h[3] << 8)) * (float)mn;
  }
  if (type == Q5_K) {
    const Q5Planes p = q5_planes(nbp);
    const uint8_t *h = w + p.hdr + tiled(row, i / 256, bpr) * 16;
    const uint32_t j = i % 256, s = j / 32, e = i % 32;
    uint32_t sc, mn;
    if (s < 4) { sc = h[4 + s] & 63u; mn = h[8 + s] & 63u; }
    else { sc = (h[8 + s] & 15u) | ((h[s] >> 6) << 4); mn = (h[8 + s] >> 4) | ((h[4 + s] >> 6) << 4); }
    const uint8_t *qh = w + p.qh + tiled(row, i / 32, cols / 32) * 4;
    const uint32_t bit = e < 16 ? 8 * (e % 4) + e / 4 : 8 * ((e - 16) % 4) + 4 + (e - 16) / 4;
    const uint32_t q = q4_quant(w, row, cols / 32, i) | (((qh[bit / 8] >> (bit % 8)) & 1u) << 4);
    return half_bits(h[0] | ((uint32_t)h[1] << 8)) * (float)(sc * q) - half_bits(h[2] | ((uint32_t)h[3] << 8)) * (float)mn;
  }
  if (type == Q4_0) {
    const uint64_t d = q40_planes(nbp).d + tiled(row, i / 32, bpr) * 2;
    return half_bits(w[d] | ((uint32_t)w[d + 1] << 8)) * (float)((int)q4_quant(w, row, cols / 32, i) - 8);
  }
  if (type == Q6_K) {
    const Q6Planes p = q6_planes(nbp);
    const uint32_t C = cols / 32;
    const float sc = (float)(int8_t)w[p.sc + tiled(row, i / 32, C) * 2 + (i % 32) / 16];
    const uint64_t d = p.d + tiled(row, i / 256, bpr) * 2;
    return half_bits(w[d] | ((uint32_t)w[d + 1] << 8)) * sc * (float)((int)q6_quant(w, nbp, row, C, i) - 32);
  }
  const Q8Planes p = q8_planes(nbp);
  const uint64_t d = p.d + tiled(row, i / 32, bpr) * 2;
  return half_bits(w[d] | ((uint32_t)w[d + 1] << 8)) * (float)(int8_t)w[p.qs + tiled(row, i / 16, cols / 16) * 16 + i % 16];
}

__global__ void k_embed_planar(int type, const uint8_t *table, uint64_t nbp, uint32_t bpr, const int32_t *ids, float *out,
                               uint32_t hidden, double scale) {
  uint32_t b = blockIdx.y, row = (uint32_t)ids[b];
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
    float v = deq_planar(type, table, nbp, bpr, hidden, row, i);
    out[(uint64_t)b * hidden + i] = scale == 1.0 ? v : (float)((double)v * scale);
  }
}

hipError_t embed_matrix(hipStream_t s, const Matrix &t, const int32_t *ids, float *out, uint32_t n, double scale) {
  if (t.layout == LAYOUT_GGUF) return embed(s, t.type, t.data, ids, out, t.cols, n, scale);
  if (!n) return hipSuccess;
  uint32_t gx = (t.cols + 255) / 256; if (gx > 64) gx = 64;
  uint32_t bpr = t.cols / block_size(t.type);
  hipLaunchKernelGGL(k_embed_planar, dim3(gx, n), dim3(256), 0, s, t.type, t.data, (uint64_t)bpr * tile_rows(t.rows), bpr,
                     ids, out, t.cols, scale);
  return hipGetLastError();
}

// ------------------------------------------------------------------ decode token start

// Workgroups 0 .. ceil(hidden / 256) - 1 gather and quantize 256 elements each (every lane of
// a 16-lane row takes part in the quantization); the last workgroup forms the rotation tables.
__global__ __launch_bounds__(256) void k_token_start(Matrix embd, uint32_t bpr, uint64_t rb, const int32_t *token, const int32_t *pos,
                                                     double scale, float *hidden, const float *norm_w, QXOut q,
                                                     RopeTables rt) {
  const uint32_t H = embd.cols;
  if (blockIdx.x == gridDim.x - 1) {
    const double p = (double)*pos;
    for (uint32_t t = 0; t < rt.n; t++)
      for (uint32_t i = threadIdx.x; i < rt.half; i += blockDim.x) {
        double sd, cd;
        sincos(p * (double)rt.scale[t] * rt.freq[t][i], &sd, &cd);
        rt.out[t][i] = (float)cd;
        rt.out[t][rt.half + i] = (float)sd;
      }
    return;
  }
  const uint32_t row = (uint32_t)*token, i = blockIdx.x * 256 + threadIdx.x;
  const bool live = i < H;
  float v = 0.f;
  if (live) {
    v = embd.layout == LAYOUT_PLANAR ? deq_planar(embd.type, embd.data, (uint64_t)bpr * tile_rows(embd.rows), bpr, H, row, i)
                                     : deq_elem(embd.type, embd.data + (uint64_t)row * rb, i);
    if (scale != 1.0) v = (float)((double)v * scale);
    hidden[i] = v;
  }
  qx_store(q, i, live && norm_w ? v * norm_w[i] : v, v, live);
}

hipError_t token_start(hipStream_t s, const Matrix &embd, const int32_t *token, const int32_t *pos, double scale,
                       float *hidden, const float *norm_w, const QXOut &q, const RopeTables &rt) {
  if (!embd.cols || embd.cols % 16 || rt.n > 2 || (rt.n && (!pos || !rt.half))) return hipErrorInvalidValue;
  const uint32_t bpr = embd.cols / block_size(embd.type);
  hipLaunchKernelGGL(k_token_start, dim3((embd.cols + 255) / 256 + 1), dim3(256), 0, s, embd, bpr,
                     row_bytes(embd.type, embd.cols), token, pos, scale,
                     hidden, norm_w, q, rt);
  return hipGetLastError();
}

// ------------------------------------------------------------------ planar repack

bool has_planar(int type, uint64_t cols) {
  if (type == Q4_K || type == Q5_K || type == Q6_K) return cols % 256 == 0;
  return (type == Q8_0 || type == Q4_0) && cols % 64 == 0;
}

uint64_t planar_bytes(int type, uint32_t cols, uint32_t rows) { return tile_rows(rows) * row_bytes(type, cols); }

// One thread per GGUF block (row, b). Q4_K: chunk c = 8b + j byte i = q[32j + i] | q[32j + 16 + i]
// << 4, with q[e] the block's quant of element e (byte 16 + 32*(e/64) + e%32, nibble
// (e%64)/32); the 16-byte header copied.
__global__ void k_repack_q4(const uint8_t *src, uint8_t *dst, uint32_t bpr, uint32_t rows) {
  const uint64_t nb = (uint64_t)rows * bpr, nbp = tile_rows(rows) * bpr;
  const uint32_t C = bpr * 8;
  const Q4Planes p = q4_planes(nbp);
  for (uint64_t blk = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; blk < nb; blk += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(blk / bpr), b = (uint32_t)(blk % bpr);
    const uint8_t *s = src + blk * 144;
    uint8_t *h = dst + p.hdr + tiled(row, b, bpr) * 16;
    for (int o = 0; o < 16; o++) h[o] = s[o];
    auto q = [&](uint32_t e) -> uint32_t { return (s[16 + 32 * (e / 64) + e % 32] >> (4 * ((e % 64) / 32))) & 15u; };
    for (uint32_t j = 0; j < 8; j++) {
      uint8_t *c = dst + p.qs + tiled(row, 8 * b + j, C) * 16;
      for (uint32_t i = 0; i < 16; i++) c[i] = (uint8_t)(q(32 * j + i) | (q(32 * j + 16 + i) << 4));
    }
  }
}

// Q6_K: ql chunk byte i = lo4[32j + i] | lo4[32j + 16 + i] << 4; qh chunk dword m byte b = hi2 of
// elements 32j + {8m+b, 16+8m+b, 8m+4+b, 16+8m+4+b} at bits 0, 2, 4, 6; the chunk's two scales;
// d per block (GGUF element e: lo4 from ql[64(e/128) + 32((e%128/32)&1) + e%32] >> 4((e%128/32)>>1),
// hi2 from qh[32(e/128) + e%32] >> 2(e%128/32)).
__global__ void k_repack_q6(const uint8_t *src, uint8_t *dst, uint32_t bpr, uint32_t rows) {
  const uint64_t nb = (uint64_t)rows * bpr, nbp = tile_rows(rows) * bpr;
  const uint32_t C = bpr * 8;
  const Q6Planes p = q6_planes(nbp);
  for (uint64_t blk = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; blk < nb; blk += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(blk / bpr), b = (uint32_t)(blk % bpr);
    const uint8_t *s = src + blk * 210;
    auto lo4 = [&](uint32_t e) -> uint32_t {
      const uint32_t h = e / 128, t = (e % 128) / 32, l = e % 32;
      return (s[64 * h + 32 * (t & 1) + l] >> (4 * (t >> 1))) & 15u;
    };
    auto hi2 = [&](uint32_t e) -> uint32_t {
      const uint32_t h = e / 128, t = (e % 128) / 32, l = e % 32;
      return (s[128 + 32 * h + l] >> (2 * t)) & 3u;
    };
    for (uint32_t j = 0; j < 8; j++) {
      const uint64_t ci = tiled(row, 8 * b + j, C);
      for (uint32_t i = 0; i < 16; i++) dst[p.ql + ci * 16 + i] = (uint8_t)(lo4(32 * j + i) | (lo4(32 * j + 16 + i) << 4));
      for (uint32_t m = 0; m < 2; m++)
        for (uint32_t bb = 0; bb < 4; bb++) {
          const uint32_t e = 32 * j + 8 * m + bb;
          dst[p.qh + ci * 8 + 4 * m + bb] = (uint8_t)(hi2(e) | (hi2(e + 16) << 2) | (hi2(e + 4) << 4) | (hi2(e + 20) << 6));
        }
      dst[p.sc + ci * 2] = s[192 + 2 * j];
      dst[p.sc + ci * 2 + 1] = s[192 + 2 * j + 1];
    }
    const uint64_t d = p.d + tiled(row, b, bpr) * 2;
    dst[d] = s[208];
    dst[d + 1] = s[209];
  }
}

// Q8_0: the 32 quants as two 16-element chunks, d per block.
__global__ void k_repack_q8(const uint8_t *src, uint8_t *dst, uint32_t bpr, uint32_t rows) {
  const uint64_t nb = (uint64_t)rows * bpr, nbp = tile_rows(rows) * bpr;
  const uint32_t C = bpr * 2;
  const Q8Planes p = q8_planes(nbp);
  for (uint64_t blk = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; blk < nb; blk += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(blk / bpr), b = (uint32_t)(blk % bpr);
    const uint8_t *s = src + blk * 34;
    const uint64_t d = p.d + tiled(row, b, bpr) * 2;
    dst[d] = s[0];
    dst[d + 1] = s[1];
    for (uint32_t h = 0; h < 2; h++)
      for (uint32_t i = 0; i < 16; i++) dst[p.qs + tiled(row, 2 * b + h, C) * 16 + i] = s[2 + 16 * h + i];
  }
}

// Q5_K: the low nibbles as Q4_K's chunks (GGUF quant bytes at 48); the fifth bits (bit e / 32
// of GGUF byte 16 + e % 32) as one dword per chunk, element e < 16 at bit 8 (e % 4) + e / 4 and
// element 16 + e at bit 8 (e % 4) + 4 + e / 4, so the bits of four consecutive elements sit
// at the same position of four bytes; the 16-byte header (d, dmin, scales) copied.
__device__ __forceinline__ uint32_t q5_bit_pos(uint32_t e) {
  return e < 16 ? 8 * (e % 4) + e / 4 : 8 * ((e - 16) % 4) + 4 + (e - 16) / 4;
}
__global__ void k_repack_q5(const uint8_t *src, uint8_t *dst, uint32_t bpr, uint32_t rows) {
  const uint64_t nb = (uint64_t)rows * bpr, nbp = tile_rows(rows) * bpr;
  const uint32_t C = bpr * 8;
  const Q5Planes p = q5_planes(nbp);
  for (uint64_t blk = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; blk < nb; blk += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(blk / bpr), b = (uint32_t)(blk % bpr);
    const uint8_t *s = src + blk * 176;
    uint8_t *h = dst + p.hdr + tiled(row, b, bpr) * 16;
    for (int o = 0; o < 16; o++) h[o] = s[o];
    auto q = [&](uint32_t e) -> uint32_t { return (s[48 + 32 * (e / 64) + e % 32] >> (4 * ((e % 64) / 32))) & 15u; };
    for (uint32_t j = 0; j < 8; j++) {
      const uint64_t ci = tiled(row, 8 * b + j, C);
      for (uint32_t i = 0; i < 16; i++) dst[p.qs + ci * 16 + i] = (uint8_t)(q(32 * j + i) | (q(32 * j + 16 + i) << 4));
      uint32_t v = 0;
      for (uint32_t e = 0; e < 32; e++) v |= ((s[16 + e] >> j) & 1u) << q5_bit_pos(e);
      for (uint32_t o = 0; o < 4; o++) dst[p.qh + ci * 4 + o] = (uint8_t)(v >> (8 * o));
    }
  }
}

// Q4_0: a block is one chunk whose GGUF quant bytes are already in chunk order (byte i holds
// elements i and i + 16); d per block.
__global__ void k_repack_q40(const uint8_t *src, uint8_t *dst, uint32_t bpr, uint32_t rows) {
  const uint64_t nb = (uint64_t)rows * bpr, nbp = tile_rows(rows) * bpr;
  const Q40Planes p = q40_planes(nbp);
  for (uint64_t blk = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; blk < nb; blk += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(blk / bpr), b = (uint32_t)(blk % bpr);
    const uint8_t *s = src + blk * 18;
    const uint64_t ci = tiled(row, b, bpr);
    dst[p.d + ci * 2] = s[0];
    dst[p.d + ci * 2 + 1] = s[1];
    for (uint32_t i = 0; i < 16; i++) dst[p.qs + ci * 16 + i] = s[2 + i];
  }
}

hipError_t repack_planar(hipStream_t s, int type, const uint8_t *src, uint8_t *dst, uint32_t cols, uint32_t rows) {
  if (!rows || !cols) return hipSuccess;
  if (!has_planar(type, cols) || cols % block_size(type)) return hipErrorInvalidValue;
  const uint32_t bpr = cols / block_size(type);
  uint64_t grid = ((uint64_t)rows * bpr + 255) / 256;
  if (grid > 65535 * 8) grid = 65535 * 8;
  if (type == Q4_K) hipLaunchKernelGGL(k_repack_q4, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, bpr, rows);
  else if (type == Q5_K) hipLaunchKernelGGL(k_repack_q5, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, bpr, rows);
  else if (type == Q6_K) hipLaunchKernelGGL(k_repack_q6, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, bpr, rows);
  else if (type == Q4_0) hipLaunchKernelGGL(k_repack_q40, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, bpr, rows);
  else hipLaunchKernelGGL(k_repack_q8, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, bpr, rows);
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

// ------------------------------------------------------------------ device properties

static int g_cus = 0;
int device_cu_count() {
  if (!g_cus) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) == hipSuccess) g_cus = p.multiProcessorCount;
    if (g_cus <= 0) g_cus = 256;
  }
  return g_cus;
}

void lds_opt_in(const void *kernel) {
  static std::mutex mu;
  static std::unordered_set<const void *> done;
  std::lock_guard<std::mutex> lock(mu);
  if (done.insert(kernel).second)
    (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_MAX);
}

hipError_t matmul(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                  uint32_t row_base, uint32_t input_offset, uint32_t batch, GemmScratch *scratch, bool accumulate) {
  if (!w.rows || !batch) return hipSuccess;
  if ((batch > 4 || w.layout != LAYOUT_GGUF) && w.cols % 64 == 0)
    return gemm(s, w, x, y, stride, row_base, input_offset, batch, scratch, accumulate);
  if (accumulate) return hipErrorInvalidValue;
  return matmul_generic(s, w, x, y, stride, row_base, input_offset, batch);
}

}  // namespace wgd
