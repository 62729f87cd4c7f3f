// gemm.hip — prompt-batch dequant-GEMM on bf16 MFMA (gfx950).
//
// The batched form of matmulShader (src/core/shaders.ts:39-54, dispatched with
// batch = prompt chunk by engine.ts:130): y[b*stride + rowBase + r] = sum_c W[r][c] x[b+off][c].
// It is a real dense contraction, so it runs on v_mfma_f32_16x16x32_bf16. bf16 keeps 8
// significant bits, which alone would cost ~2^-9 relative error per output and break the
// 1e-3 logits bound, so both operands are split: v = hi + lo with hi = RN_bf16(v),
// lo = RN_bf16(v - hi), and the product is accumulated as hi*hi + hi*lo + lo*hi in f32
// (relative error ~2^-16). Weights are dequantized from their GGUF (or planar) blocks
// straight into MFMA operand registers; the activation tile is split once into LDS.
//
// Tiling: a workgroup (4 wavefronts) owns 64 rows x 64 tokens; each wavefront owns
// 16 rows x 64 tokens = four 16x16 accumulator tiles; K advances 32 per MFMA step and
// 64 per LDS tile.
#include "internal.h"
#include "decode.h"

namespace wgd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Round-to-nearest-even f32 -> bf16 bits (finite inputs).
__device__ __forceinline__ uint32_t bf16_rne(float v) {
  uint32_t b = __float_as_uint(v);
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ void split8(const float *v, uint4 &hi, uint4 &lo) {
  uint32_t h[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    h[i] = bf16_rne(v[i]);
    l[i] = bf16_rne(v[i] - __uint_as_float(h[i] << 16));
  }
  hi = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
  lo = make_uint4(l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16), l[6] | (l[7] << 16));
}

struct GemmArgs {
  const uint8_t *w; int type, layout;
  uint64_t rb, nbt; uint32_t bpr;
  const float *x; float *y;
  uint32_t cols, rows, stride, row_base, input_offset, batch;
};

// Eight consecutive weights w[row][k .. k+8) (k % 8 == 0) as f32.
__device__ __forceinline__ void load_a8(const GemmArgs &a, uint32_t row, uint32_t k, float *o) {
  if (a.type == Q4_K && a.layout == LAYOUT_GGUF) {
    const uint8_t *blk = a.w + (uint64_t)row * a.rb + (uint64_t)(k >> 8) * 144;
    uint32_t j = k & 255, s = j >> 5, l0 = j & 31;
    uint4 h = *(const uint4 *)blk;
    uint2 qv = *(const uint2 *)(blk + 16 + (s >> 1) * 32 + l0);
    uint32_t A = h.y, B = h.z, C = h.w, sh = 8 * (s & 3), sc, m;
    if (s < 4) { sc = (A >> sh) & 63u; m = (B >> sh) & 63u; }
    else { sc = ((C >> sh) & 15u) | (((A >> sh) >> 6 & 3u) << 4); m = ((C >> sh) >> 4 & 15u) | (((B >> sh) >> 6 & 3u) << 4); }
    float dsc = half_bits(h.x & 0xFFFFu) * (float)sc, dmm = half_bits(h.x >> 16) * (float)m;
    uint32_t sq = 4 * (s & 1);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t byte = ((i < 4 ? qv.x : qv.y) >> (8 * (i & 3))) & 0xFFu;
      o[i] = dsc * (float)((byte >> sq) & 15u) - dmm;
    }
    return;
  }
  if (a.type == Q4_K && a.layout == LAYOUT_PLANAR) {
    const Q4Planes p = q4_planes(a.nbt);
    const uint32_t j = k & 255, s = j >> 5, e0 = k & 31;
    uint4 h = *(const uint4 *)(a.w + p.hdr + tiled(row, k >> 8, a.bpr) * 16);
    // chunk k / 32, bytes e0 % 16 .. +8, nibble e0 / 16
    uint2 qv = *(const uint2 *)(a.w + p.qs + tiled(row, k >> 5, a.bpr * 8) * 16 + (e0 & 15));
    uint32_t A = h.y, B = h.z, C = h.w, sh = 8 * (s & 3), sc, m;
    if (s < 4) { sc = (A >> sh) & 63u; m = (B >> sh) & 63u; }
    else { sc = ((C >> sh) & 15u) | (((A >> sh) >> 6 & 3u) << 4); m = ((C >> sh) >> 4 & 15u) | (((B >> sh) >> 6 & 3u) << 4); }
    float dsc = half_bits(h.x & 0xFFFFu) * (float)sc, dmm = half_bits(h.x >> 16) * (float)m;
    uint32_t sq = 4 * (e0 >> 4);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t byte = ((i < 4 ? qv.x : qv.y) >> (8 * (i & 3))) & 0xFFu;
      o[i] = dsc * (float)((byte >> sq) & 15u) - dmm;
    }
    return;
  }
  if (a.type == Q6_K && a.layout == LAYOUT_PLANAR) {
    const Q6Planes p = q6_planes(a.nbt);
    const uint32_t e0 = k & 31, h = e0 >> 4;
    const uint64_t ci = tiled(row, k >> 5, a.bpr * 8);
    uint2 lo = *(const uint2 *)(a.w + p.ql + ci * 16 + (e0 & 15));
    // high bits of elements e0 .. e0+7: qh dword (e0 % 16) / 8, byte i % 4, bit 4 * (i / 4) + 2h
    uint32_t hq = *(const uint32_t *)(a.w + p.qh + ci * 8 + 4 * ((e0 & 15) >> 3));
    float sc = (float)(int8_t)a.w[p.sc + ci * 2 + h];
    float d = half_bits(*(const uint16_t *)(a.w + p.d + tiled(row, k >> 8, a.bpr) * 2)) * sc;
    uint32_t ls = 4 * h;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t lb = ((i < 4 ? lo.x : lo.y) >> (8 * (i & 3))) & 0xFFu;
      uint32_t hb = (hq >> (8 * (i & 3) + 4 * (i >> 2) + 2 * h)) & 3u;
      o[i] = d * (float)((int)(((lb >> ls) & 15u) | (hb << 4)) - 32);
    }
    return;
  }
  if (a.type == Q8_0 && a.layout == LAYOUT_PLANAR) {
    const Q8Planes p = q8_planes(a.nbt);
    uint2 q = *(const uint2 *)(a.w + p.qs + tiled(row, k >> 4, a.bpr * 2) * 16 + (k & 15));
    float d = half_bits(*(const uint16_t *)(a.w + p.d + tiled(row, k >> 5, a.bpr) * 2));
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = d * (float)(int8_t)(((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu);
    return;
  }
  const uint8_t *r = a.w + (uint64_t)row * a.rb;
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = deq_elem(a.type, r, k + i);
}

constexpr int KT = 64;              // K per LDS tile
constexpr int NT = 64;              // tokens per workgroup
constexpr int XPITCH = KT + 8;      // bf16 elements per LDS row (16-byte pad)

__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t xh[NT * XPITCH];
  __shared__ __attribute__((aligned(16))) uint16_t xl[NT * XPITCH];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t m0 = blockIdx.x * 64 + wv * 16, n0 = blockIdx.y * NT;
  const uint32_t arow = m0 + (lane & 15), kg = 8 * (lane >> 4);
  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (uint32_t k0 = 0; k0 < a.cols; k0 += KT) {
    // Stage x[n0 .. n0+64)[k0 .. k0+64) as split bf16: 256 threads x 16 elements.
    {
      uint32_t n = tid >> 2, kk = (tid & 3) * 16;
      float v[16];
      if (n0 + n < a.batch && k0 + kk < a.cols) {
        const float4 *src = (const float4 *)(a.x + (uint64_t)(n0 + n + a.input_offset) * a.cols + k0 + kk);
#pragma unroll
        for (int i = 0; i < 4; i++) { float4 t = src[i]; v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w; }
      } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = 0.f;
      }
      uint4 h0, l0, h1, l1;
      split8(v, h0, l0); split8(v + 8, h1, l1);
      *(uint4 *)&xh[n * XPITCH + kk] = h0; *(uint4 *)&xh[n * XPITCH + kk + 8] = h1;
      *(uint4 *)&xl[n * XPITCH + kk] = l0; *(uint4 *)&xl[n * XPITCH + kk + 8] = l1;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < KT; ks += 32) {
      float wv8[8];
      if (arow < a.rows) load_a8(a, arow, k0 + ks + kg, wv8);
      else {
#pragma unroll
        for (int i = 0; i < 8; i++) wv8[i] = 0.f;
      }
      uint4 ah, al;
      split8(wv8, ah, al);
      bf16x8 Ah = __builtin_bit_cast(bf16x8, ah), Al = __builtin_bit_cast(bf16x8, al);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        uint32_t n = t * 16 + (lane & 15);
        bf16x8 Bh = __builtin_bit_cast(bf16x8, *(const uint4 *)&xh[n * XPITCH + ks + kg]);
        bf16x8 Bl = __builtin_bit_cast(bf16x8, *(const uint4 *)&xl[n * XPITCH + ks + kg]);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bh, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bl, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Bh, acc[t], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // D layout: lane holds rows 4*(lane/16)+i, token column lane%16 of each 16x16 tile.
#pragma unroll
  for (int t = 0; t < 4; t++) {
    uint32_t tok = n0 + t * 16 + (lane & 15);
    if (tok >= a.batch) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t row = m0 + 4 * (lane >> 4) + i;
      if (row < a.rows) a.y[(uint64_t)tok * a.stride + a.row_base + row] = acc[t][i];
    }
  }
}

hipError_t gemm(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                uint32_t row_base, uint32_t input_offset, uint32_t batch) {
  if (!w.rows || !batch) return hipSuccess;
  if (w.cols % KT) return hipErrorInvalidValue;
  GemmArgs a;
  a.w = w.data; a.type = w.type; a.layout = w.layout;
  a.rb = row_bytes(w.type, w.cols); a.bpr = w.cols / block_size(w.type);
  a.nbt = (uint64_t)a.bpr * (w.layout == LAYOUT_PLANAR ? tile_rows(w.rows) : w.rows);
  a.x = x; a.y = y; a.cols = w.cols; a.rows = w.rows; a.stride = stride; a.row_base = row_base;
  a.input_offset = input_offset; a.batch = batch;
  dim3 grid((w.rows + 63) / 64, (batch + NT - 1) / NT);
  hipLaunchKernelGGL(k_gemm, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace wgd
