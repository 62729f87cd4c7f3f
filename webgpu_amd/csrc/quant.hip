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

// Gather from a planar table: element i of `row`, decoded exactly as deq_elem.
__device__ __forceinline__ float deq_planar(int type, const uint8_t *w, uint64_t nbt, uint32_t bpr, uint32_t row, uint32_t i) {
  const uint64_t bi = (uint64_t)row * bpr + i / block_size_dev(type);
  if (type == Q4_K) {
    const uint8_t *h = w + q4_planes(nbt).hdr + bi * 16;
    const uint32_t j = i % 256, s = j / 32, e = j % 32;
    uint32_t sc, mn;
    if (s < 4) { sc = h[4 + s] & 63u; mn = h[8 + s] & 63u; }
    else { sc = (h[8 + s] & 15u) | ((h[s] >> 6) << 4); mn = (h[8 + s] >> 4) | ((h[4 + s] >> 6) << 4); }
    const uint32_t q = q4_quant(w, bi * 8 + s, e);
    return half_bits(h[0] | ((uint32_t)h[1] << 8)) * (float)(sc * q) - half_bits(h[2] | ((uint32_t)h[3] << 8)) * (float)mn;
  }
  if (type == Q6_K) {
    const Q6Planes p = q6_planes(nbt);
    const uint32_t j = i % 256, s = j / 32, e = j % 32;
    const uint64_t ci = bi * 8 + s;
    const float sc = (float)(int8_t)w[p.sc + ci * 2 + e / 16];
    return half_bits(w[p.d + bi * 2] | ((uint32_t)w[p.d + bi * 2 + 1] << 8)) * sc * (float)((int)q6_quant(w, nbt, ci, e) - 32);
  }
  const Q8Planes p = q8_planes(nbt);
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

bool has_planar(int type) { return type == Q4_K || type == Q6_K || type == Q8_0; }

// One thread per block. Q4_K: chunk j (sub-block j) byte i = q[32j + i] | q[32j + 16 + i] << 4,
// with q[e] the GGUF quant of element e (byte 16 + 32*(e/64) + e%32, nibble (e%64)/32).
__global__ void k_repack_q4(const uint8_t *src, uint8_t *dst, uint64_t nb) {
  const Q4Planes p = q4_planes(nb);
  for (uint64_t blk = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; blk < nb; blk += (uint64_t)gridDim.x * blockDim.x) {
    const uint8_t *b = src + blk * 144;
    for (int o = 0; o < 16; o++) dst[p.hdr + blk * 16 + o] = b[o];
    auto q = [&](uint32_t e) -> uint32_t { return (b[16 + 32 * (e / 64) + e % 32] >> (4 * ((e % 64) / 32))) & 15u; };
    for (uint32_t j = 0; j < 8; j++)
      for (uint32_t i = 0; i < 16; i++) dst[p.qs + blk * 128 + 16 * j + i] = (uint8_t)(q(32 * j + i) | (q(32 * j + 16 + i) << 4));
  }
}

// Q6_K: ql chunk j byte i = lo4[32j + i] | lo4[32j + 16 + i] << 4; qh chunk j dword m byte b =
// hi2 of elements 32j + {8m+b, 16+8m+b, 8m+4+b, 16+8m+4+b} at bits 0, 2, 4, 6; scales and d
// copied (GGUF element e: lo4 from ql[64(e/128) + 32((e%128/32)&1) + e%32] >> 4((e%128/32)>>1),
// hi2 from qh[32(e/128) + e%32] >> 2(e%128/32)).
__global__ void k_repack_q6(const uint8_t *src, uint8_t *dst, uint64_t nb) {
  const Q6Planes p = q6_planes(nb);
  for (uint64_t blk = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; blk < nb; blk += (uint64_t)gridDim.x * blockDim.x) {
    const uint8_t *b = src + blk * 210;
    auto lo4 = [&](uint32_t e) -> uint32_t {
      const uint32_t h = e / 128, t = (e % 128) / 32, l = e % 32;
      return (b[64 * h + 32 * (t & 1) + l] >> (4 * (t >> 1))) & 15u;
    };
    auto hi2 = [&](uint32_t e) -> uint32_t {
      const uint32_t h = e / 128, t = (e % 128) / 32, l = e % 32;
      return (b[128 + 32 * h + l] >> (2 * t)) & 3u;
    };
    for (uint32_t j = 0; j < 8; j++) {
      for (uint32_t i = 0; i < 16; i++) dst[p.ql + blk * 128 + 16 * j + i] = (uint8_t)(lo4(32 * j + i) | (lo4(32 * j + 16 + i) << 4));
      for (uint32_t m = 0; m < 2; m++)
        for (uint32_t bb = 0; bb < 4; bb++) {
          const uint32_t e = 32 * j + 8 * m + bb;
          dst[p.qh + blk * 64 + 8 * j + 4 * m + bb] =
              (uint8_t)(hi2(e) | (hi2(e + 16) << 2) | (hi2(e + 4) << 4) | (hi2(e + 20) << 6));
        }
    }
    for (int o = 0; o < 16; o++) dst[p.sc + blk * 16 + o] = b[192 + o];
    dst[p.d + blk * 2] = b[208];
    dst[p.d + blk * 2 + 1] = b[209];
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
  if (type != Q8_0) { grid = (blocks + 255) / 256; if (grid > 65535 * 8) grid = 65535 * 8; }
  if (type == Q4_K) hipLaunchKernelGGL(k_repack_q4, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, blocks);
  else if (type == Q6_K) hipLaunchKernelGGL(k_repack_q6, dim3((uint32_t)grid), dim3(256), 0, s, src, dst, blocks);
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

hipError_t matmul(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                  uint32_t row_base, uint32_t input_offset, uint32_t batch) {
  if (!w.rows || !batch) return hipSuccess;
  if ((batch > 4 || w.layout != LAYOUT_GGUF) && w.cols % 64 == 0)
    return gemm(s, w, x, y, stride, row_base, input_offset, batch);
  return matmul_generic(s, w, x, y, stride, row_base, input_offset, batch);
}

}  // namespace wgd
