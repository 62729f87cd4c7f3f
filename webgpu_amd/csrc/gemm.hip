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
#include "split.h"

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
  if (a.type == Q5_K && a.layout == LAYOUT_PLANAR) {
    const Q5Planes p = q5_planes(a.nbt);
    const uint32_t j = k & 255, s = j >> 5, e0 = k & 31;
    uint4 h = *(const uint4 *)(a.w + p.hdr + tiled(row, k >> 8, a.bpr) * 16);
    uint2 qv = *(const uint2 *)(a.w + p.qs + tiled(row, k >> 5, a.bpr * 8) * 16 + (e0 & 15));
    const uint32_t hb = *(const uint32_t *)(a.w + p.qh + tiled(row, k >> 5, a.bpr * 8) * 4);
    uint32_t A = h.y, B = h.z, C = h.w, sh = 8 * (s & 3), sc, m;
    if (s < 4) { sc = (A >> sh) & 63u; m = (B >> sh) & 63u; }
    else { sc = ((C >> sh) & 15u) | (((A >> sh) >> 6 & 3u) << 4); m = ((C >> sh) >> 4 & 15u) | (((B >> sh) >> 6 & 3u) << 4); }
    float dsc = half_bits(h.x & 0xFFFFu) * (float)sc, dmm = half_bits(h.x >> 16) * (float)m;
    uint32_t sq = 4 * (e0 >> 4);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      // fifth bit of chunk element e: byte e % 4, bit e / 4 (e < 16) or 4 + (e - 16) / 4
      const uint32_t e = e0 + i, pos = 8 * (e & 3) + (e < 16 ? e / 4 : 4 + (e - 16) / 4);
      uint32_t byte = ((i < 4 ? qv.x : qv.y) >> (8 * (i & 3))) & 0xFFu;
      o[i] = dsc * (float)(((byte >> sq) & 15u) | (((hb >> pos) & 1u) << 4)) - dmm;
    }
    return;
  }
  if (a.type == Q4_0 && a.layout == LAYOUT_PLANAR) {
    const Q40Planes p = q40_planes(a.nbt);
    const uint32_t e0 = k & 31;
    uint2 qv = *(const uint2 *)(a.w + p.qs + tiled(row, k >> 5, a.bpr) * 16 + (e0 & 15));
    float d = half_bits(*(const uint16_t *)(a.w + p.d + tiled(row, k >> 5, a.bpr) * 2));
    uint32_t sq = 4 * (e0 >> 4);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t byte = ((i < 4 ? qv.x : qv.y) >> (8 * (i & 3))) & 0xFFu;
      o[i] = d * (float)((int)((byte >> sq) & 15u) - 8);
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
  if (a.type == F16 && (a.rb & 15) == 0) {
    // eight halves in one 16-byte load (rows stay 16-byte aligned for K % 8 == 0)
    const uint4 v = *(const uint4 *)(r + 2 * (uint64_t)k);
    const uint32_t h[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      o[2 * i] = half_bits(h[i] & 0xFFFFu);
      o[2 * i + 1] = half_bits(h[i] >> 16);
    }
    return;
  }
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

// ------------------------------------------------------------------ planar K-quant GEMM
//
// The prompt GEMM of the planar layouts (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0; the decode matvec's weights). A
// workgroup owns QG_M = 128 weight rows x QG_N = 128 tokens and a K span (split-K when the
// rows alone give too few workgroups; partial sums are added in split order by
// k_gemm_reduce, so results do not depend on timing). The activations are split into bf16
// (hi, lo) once per input by k_gemm_split, already in MFMA fragment order, so each
// wavefront loads its activation fragments of a K tile straight from that buffer (L2
// hits: every workgroup of the launch reads the same tiles) into registers, 1 KB per load
// instruction, before the tile's dequantization. Per 64-column K tile every weight of the
// workgroup's rows is dequantized once, from coalesced 16-byte planar loads (one 32-element
// chunk of one row per thread), split the same way and stored in LDS in fragment order.
// Four wavefronts each compute 64 rows x 64 tokens, sixteen 16 x 16 accumulators, three
// MFMAs per product (hi*hi + hi*lo + lo*hi). The next K tile's weight loads are issued
// before the MFMAs of the current one; two workgroups share a CU (the register budget of
// the launch bounds), so one's dequantization can run beside the other's MFMAs.
//
// The weight tile is kept in LDS in the activations' fragment order (split.h), as rows.
constexpr uint32_t QG_M = 128, QG_N = SPLIT_N, QG_K = SPLIT_K, QG_TILE = SPLIT_TILE;
constexpr uint32_t QG_LDS = QG_TILE * 2;  // bytes: weight tile

// One weight matrix of a grouped launch: its planar geometry, the row-tile count, and where
// its rows go (y, or rows [row0, row0 + rows) of the group's split-K partial sums).
struct QJob {
  const uint8_t *w; uint32_t wbytes;
  uint32_t C, bpr, nbp;  // chunk columns, blocks per row, blocks of the padded matrix
  uint32_t rows, tiles, kind, row0;
  float *y; uint32_t stride, row_base;
};
constexpr uint32_t QG_MAX_JOBS = 3;
// Matrices that read the same activations, launched together: workgroups (tile, split)
// over the concatenated row tiles; kind 0 / 1 selects the launch's first / second type.
struct QGemm {
  QJob job[QG_MAX_JOBS]; uint32_t njobs;
  const uint16_t *xs; float *part;
  uint32_t cols, batch, kspan, rows_total, accumulate;
};

// Activations [batch][cols] f32 -> the split form (split.h); tokens past the batch up to the
// tile are zero. One thread per eight consecutive columns of a token.
__global__ __launch_bounds__(256) void k_gemm_split(const float *x, uint16_t *xs, uint32_t cols, uint32_t batch,
                                                    uint32_t count) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const uint32_t c8 = cols / 8, tok = i / c8, k = (i % c8) * 8;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
  if (tok < batch) {
    a = *(const float4 *)(x + (uint64_t)tok * cols + k);
    b = *(const float4 *)(x + (uint64_t)tok * cols + k + 4);
  }
  split_store8(xs, cols, tok, k, a, b);
}

typedef __amdgpu_buffer_rsrc_t QRsrc;
__device__ __forceinline__ uint4 qld16(QRsrc r, uint32_t off) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// One thread's weights of a K tile: Q4_K / Q6_K one 32-element chunk (row-tile rt, column
// cc of the tile, row r), Q8_0 two 16-element chunks.
template <int TYPE> struct QWeights;
template <> struct QWeights<Q4_K> {
  uint4 q, h;
  __device__ void fetch(const QJob &a, QRsrc rw, uint32_t T, uint32_t r, uint32_t c) {
    q = qld16(rw, ((T * a.C + c) * 16 + r) * 16);
    h = qld16(rw, a.nbp * 128 + ((T * a.bpr + c / 8) * 16 + r) * 16);
  }
  // element e < 32 of the chunk into f32 (quant.ts:13-19: d * sc * q - dmin * m)
  __device__ void values(uint32_t c, float *v) const {
    const uint32_t s = c & 7, sh = 8 * (s & 3);
    uint32_t sc, m;
    if (s < 4) { sc = (h.y >> sh) & 63u; m = (h.z >> sh) & 63u; }
    else { sc = ((h.w >> sh) & 15u) | (((h.y >> sh) >> 6 & 3u) << 4); m = ((h.w >> sh) >> 4 & 15u) | (((h.z >> sh) >> 6 & 3u) << 4); }
    const float dsc = half_bits(h.x & 0xFFFFu) * (float)sc, dmm = half_bits(h.x >> 16) * (float)m;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        v[4 * k + b] = fmaf(dsc, (float)((lo >> (8 * b)) & 0xFFu), -dmm);
        v[16 + 4 * k + b] = fmaf(dsc, (float)((hi >> (8 * b)) & 0xFFu), -dmm);
      }
    }
  }
};
template <> struct QWeights<Q6_K> {
  uint4 q; uint2 qh; uint32_t sc, d;
  __device__ void fetch(const QJob &a, QRsrc rw, uint32_t T, uint32_t r, uint32_t c) {
    const uint32_t tc = (T * a.C + c) * 16 + r;
    q = qld16(rw, tc * 16);
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 hv = __builtin_amdgcn_raw_buffer_load_b64(rw, a.nbp * 128 + tc * 8, 0, 0);
    qh = make_uint2(hv.x, hv.y);
    sc = __builtin_amdgcn_raw_buffer_load_b16(rw, a.nbp * 192 + tc * 2, 0, 0);
    d = __builtin_amdgcn_raw_buffer_load_b16(rw, a.nbp * 208 + ((T * a.bpr + c / 8) * 16 + r) * 2, 0, 0);
  }
  // quant.ts:21-27: d * scale16 * (q - 32); low nibbles with high bits at bits 4-5
  __device__ void values(uint32_t, float *v) const {
    const float d0 = half_bits(d & 0xFFFFu);
    const float s0 = d0 * (float)(int8_t)(sc & 0xFFu), s1 = d0 * (float)(int8_t)((sc >> 8) & 0xFFu);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t Q = (k < 2 ? qh.x : qh.y) >> (4 * (k & 1));
      const uint32_t lo = (qw[k] & 0x0F0F0F0Fu) | ((Q << 4) & 0x30303030u);
      const uint32_t hi = ((qw[k] >> 4) & 0x0F0F0F0Fu) | ((Q << 2) & 0x30303030u);
#pragma unroll
      for (int b = 0; b < 4; b++) {
        v[4 * k + b] = s0 * (float)((int)((lo >> (8 * b)) & 0xFFu) - 32);
        v[16 + 4 * k + b] = s1 * (float)((int)((hi >> (8 * b)) & 0xFFu) - 32);
      }
    }
  }
};
template <> struct QWeights<Q8_0> {
  uint4 q[2]; uint32_t d[2];
  // chunks 2c and 2c + 1 (16 elements each, one Q8_0 block): c counts 32-element columns
  __device__ void fetch(const QJob &a, QRsrc rw, uint32_t T, uint32_t r, uint32_t c) {
#pragma unroll
    for (int u = 0; u < 2; u++) q[u] = qld16(rw, ((T * a.C + 2 * c + u) * 16 + r) * 16);
    d[0] = d[1] = __builtin_amdgcn_raw_buffer_load_b16(rw, a.nbp * 32 + ((T * a.bpr + c) * 16 + r) * 2, 0, 0);
  }
  __device__ void values(uint32_t, float *v) const {
    const float dd = half_bits(d[0] & 0xFFFFu);
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const uint32_t qw[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
      for (int k = 0; k < 4; k++)
#pragma unroll
        for (int b = 0; b < 4; b++) v[16 * u + 4 * k + b] = dd * (float)(int8_t)((qw[k] >> (8 * b)) & 0xFFu);
    }
  }
};

// Q5_K: Q4_K's chunk and header planes (the header after the fifth-bit plane) and the
// chunk's dword of fifth bits, moved to bit 4 of each quant byte (quant.ts:13-19).
template <> struct QWeights<Q5_K> {
  uint4 q, h; uint32_t b;
  __device__ void fetch(const QJob &a, QRsrc rw, uint32_t T, uint32_t r, uint32_t c) {
    const uint32_t tc = (T * a.C + c) * 16 + r;
    q = qld16(rw, tc * 16);
    b = __builtin_amdgcn_raw_buffer_load_b32(rw, a.nbp * 128 + tc * 4, 0, 0);
    h = qld16(rw, a.nbp * 160 + ((T * a.bpr + c / 8) * 16 + r) * 16);
  }
  __device__ void values(uint32_t c, float *v) const {
    const uint32_t s = c & 7, sh = 8 * (s & 3);
    uint32_t sc, m;
    if (s < 4) { sc = (h.y >> sh) & 63u; m = (h.z >> sh) & 63u; }
    else { sc = ((h.w >> sh) & 15u) | (((h.y >> sh) >> 6 & 3u) << 4); m = ((h.w >> sh) >> 4 & 15u) | (((h.z >> sh) >> 6 & 3u) << 4); }
    const float dsc = half_bits(h.x & 0xFFFFu) * (float)sc, dmm = half_bits(h.x >> 16) * (float)m;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t lo = (qw[k] & 0x0F0F0F0Fu) | ((b << (4 - k)) & 0x10101010u);
      const uint32_t hi = ((qw[k] >> 4) & 0x0F0F0F0Fu) | ((b >> k) & 0x10101010u);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[4 * k + e] = fmaf(dsc, (float)((lo >> (8 * e)) & 0xFFu), -dmm);
        v[16 + 4 * k + e] = fmaf(dsc, (float)((hi >> (8 * e)) & 0xFFu), -dmm);
      }
    }
  }
};
// Q4_0: one block per chunk, d * (q - 8) (quant.ts:7).
template <> struct QWeights<Q4_0> {
  uint4 q; uint32_t d;
  __device__ void fetch(const QJob &a, QRsrc rw, uint32_t T, uint32_t r, uint32_t c) {
    const uint32_t tc = (T * a.C + c) * 16 + r;
    q = qld16(rw, tc * 16);
    d = __builtin_amdgcn_raw_buffer_load_b16(rw, a.nbp * 16 + tc * 2, 0, 0);
  }
  __device__ void values(uint32_t, float *v) const {
    const float dd = half_bits(d & 0xFFFFu);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[4 * k + e] = dd * (float)((int)((qw[k] >> (8 * e)) & 15u) - 8);
        v[16 + 4 * k + e] = dd * (float)((int)((qw[k] >> (8 * e + 4)) & 15u) - 8);
      }
  }
};

template <int TYPE>
__device__ __forceinline__ void gemm_tile(const QGemm &a, const QJob &jb, uint32_t mt, uint16_t *qlds) {
  uint16_t *wt = qlds;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, wm = wv & 1, wn = wv >> 1;
  const uint32_t m0 = mt * QG_M, n0 = blockIdx.y * QG_N, z = blockIdx.z;
  const uint32_t kb = z * a.kspan, ke = kb + a.kspan < a.cols ? kb + a.kspan : a.cols;
  const QRsrc rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(jb.w), 0, (int)jb.wbytes, 0x00020000);
  // this thread's weights: row tile wrt, 32-column half wcc of the K tile, row wr
  const uint32_t wrt = tid >> 5, wcc = (tid >> 4) & 1, wr = tid & 15;
  const uint32_t ktiles = a.cols / QG_K;
  const QRsrc rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.xs + (uint64_t)blockIdx.y * ktiles * QG_TILE), 0, (int)(ktiles * QG_TILE * 2), 0x00020000);
  QWeights<TYPE> wreg;
  auto fetch = [&](uint32_t k0) { wreg.fetch(jb, rw, m0 / 16 + wrt, wr, k0 / 32 + wcc); };
  // this wavefront's activation fragments of a K tile, from the split buffer
  auto xfrag = [&](uint32_t k0, uint32_t hl, uint32_t b, uint32_t ks) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
        rx, 2 * ((k0 / QG_K) * QG_TILE + frag_at(hl, b, ks, 0, 0) + 8 * lane), 0, 0));
  };
  auto stage = [&](uint32_t k0) {
    float v[32];
    wreg.values(k0 / 32 + wcc, v);
    uint32_t h[16], l[16];
#pragma unroll
    for (int i = 0; i < 16; i++) split2(v[2 * i], v[2 * i + 1], h[i], l[i]);
#pragma unroll
    for (uint32_t g = 0; g < 4; g++) {
      *(uint4 *)(wt + frag_at(0, wrt, wcc, g, wr)) = make_uint4(h[4 * g], h[4 * g + 1], h[4 * g + 2], h[4 * g + 3]);
      *(uint4 *)(wt + frag_at(1, wrt, wcc, g, wr)) = make_uint4(l[4 * g], l[4 * g + 1], l[4 * g + 2], l[4 * g + 3]);
    }
  };
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  fetch(kb);
  for (uint32_t k0 = kb; k0 < ke; k0 += QG_K) {
    bf16x8 Bh[2][4], Bl[2][4];
#pragma unroll
    for (uint32_t ks = 0; ks < 2; ks++)
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) {
        Bh[ks][i] = xfrag(k0, 0, wn * 4 + i, ks);
        Bl[ks][i] = xfrag(k0, 1, wn * 4 + i, ks);
      }
    stage(k0);
    __syncthreads();
    if (k0 + QG_K < ke) fetch(k0 + QG_K);  // next tile's loads fly during the MFMAs
#pragma unroll
    for (uint32_t ks = 0; ks < 2; ks++) {
      bf16x8 Ah[4], Al[4];
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) {
        Ah[i] = *(const bf16x8 *)(wt + frag_at(0, wm * 4 + i, ks, 0, 0) + 8 * lane);
        Al[i] = *(const bf16x8 *)(wt + frag_at(1, wm * 4 + i, ks, 0, 0) + 8 * lane);
      }
      // the three products of a tile are 16 MFMAs apart (every tile's first, then second, then third)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Bh[ks][j], Ah[i], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Bl[ks][j], Ah[i], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Bh[ks][j], Al[i], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // The products are formed as X W^T, so lane (g, c) of tile (i, j) holds tokens 16 j + 4 g + e
  // of row 16 i + c: each store writes 16 consecutive rows of four tokens.
  const uint32_t row0 = m0 + wm * 64 + (lane & 15);
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t tok = n0 + wn * 64 + 16 * j + 4 * (lane >> 4) + e;
      if (tok >= a.batch) continue;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t row = row0 + 16 * i;
        if (row >= jb.rows) continue;
        if (a.part) {
          a.part[((uint64_t)z * a.batch + tok) * a.rows_total + jb.row0 + row] = acc[i][j][e];
        } else {
          float *py = jb.y + (uint64_t)tok * jb.stride + jb.row_base + row;
          *py = a.accumulate ? *py + acc[i][j][e] : acc[i][j][e];
        }
      }
    }
}

// blockIdx.x walks the jobs' row tiles in order; a job of kind 1 runs the second type.
template <int T0, int T1>
__global__ __launch_bounds__(256, 2) void k_gemm_q(QGemm a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t qlds[];
  uint32_t t = blockIdx.x, j = 0;
  while (j + 1 < a.njobs && t >= a.job[j].tiles) { t -= a.job[j].tiles; j++; }
  const QJob &jb = a.job[j];
  if (T0 == T1 || jb.kind == 0) gemm_tile<T0>(a, jb, t, qlds);
  else gemm_tile<T1>(a, jb, t, qlds);
}

// Sum of the split-K partials part[z][tok][rows_total] in split order into each job's rows
// (accumulate: added to y).
template <uint32_t S>
__global__ __launch_bounds__(256) void k_gemm_reduce(QGemm a, uint32_t splits) {
  const uint64_t n = (uint64_t)a.rows_total * a.batch;
  const __amdgpu_buffer_rsrc_t rp = split_rsrc(a.part, splits, n);
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
    const float v = split_sum<S>(rp, splits, (uint32_t)(4 * n), (uint32_t)(4 * i));
    const uint32_t tok = (uint32_t)(i / a.rows_total);
    uint32_t r = (uint32_t)(i % a.rows_total), j = 0;
    while (j + 1 < a.njobs && r >= a.job[j].rows) { r -= a.job[j].rows; j++; }
    float *py = a.job[j].y + (uint64_t)tok * a.job[j].stride + a.job[j].row_base + r;
    *py = a.accumulate ? *py + v : v;
  }
}

// The GLU finish (k_glu_reduce) of columns k .. k + 7 of token tok.
template <uint32_t S>
__device__ __forceinline__ void glu_finish8(const float *part, uint32_t splits, uint32_t R, uint32_t batch, float *y,
                                            uint16_t *xs, int act, const DeferredNorm &dn, uint32_t tok, uint32_t k) {
  const uint64_t n = (uint64_t)2 * R * batch, row = (uint64_t)tok * 2 * R;
  const __amdgpu_buffer_rsrc_t rp = split_rsrc(part, splits, n);
  const uint32_t sb = (uint32_t)(4 * n), og = (uint32_t)(4 * (row + k)), ou = og + 4 * R;
  const float4 g0 = split_sum4<S>(rp, splits, sb, og), g1 = split_sum4<S>(rp, splits, sb, og + 16);
  const float4 u0 = split_sum4<S>(rp, splits, sb, ou), u1 = split_sum4<S>(rp, splits, sb, ou + 16);
  float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
  if (dn.sq) {
    const float xinv = deferred_inv(dn, tok);
#pragma unroll
    for (int e = 0; e < 8; e++) { g[e] *= xinv; u[e] *= xinv; }
  }
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = glu_act(g[e], act) * u[e];
  const float4 a = make_float4(v[0], v[1], v[2], v[3]), b = make_float4(v[4], v[5], v[6], v[7]);
  if (y) {
    *(float4 *)(y + (uint64_t)tok * R + k) = a;
    *(float4 *)(y + (uint64_t)tok * R + k + 4) = b;
  }
  split_store8(xs, R, tok, k, a, b);
}

// gate (rows [0, R)) and up (rows [R, 2R)) from the split-K partials, then act(gate) * up
// into y [batch][R] and its split form for the down GEMM: one thread per eight columns of a
// token. S >= splits.
//
// The GEMM's 128-row tile t ran on XCD t % 8 (its grid's first dimension, the tile count, is
// a multiple of 8, and workgroups go to the XCDs round-robin), and with R a multiple of 1024
// the up tile of a column has the gate tile's residue. Then (by_xcd) workgroup w, on XCD
// w % 8, takes token w / 8 and the columns of the tiles t = w (mod 8), reading only
// partials its XCD wrote: each 128-row run of the scratch stays with one XCD, and the next
// GEMM's writes to it take no coherence probes. Otherwise workgroup w takes 256
// consecutive column groups.
template <uint32_t S>
__global__ __launch_bounds__(256) void k_glu_reduce(const float *part, uint32_t splits, uint32_t R, uint32_t batch,
                                                    float *y, uint16_t *xs, int act, DeferredNorm dn, uint32_t by_xcd) {
  if (!by_xcd) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < batch * (R / 8)) glu_finish8<S>(part, splits, R, batch, y, xs, act, dn, i / (R / 8), (i % (R / 8)) * 8);
    return;
  }
  const uint32_t x = blockIdx.x % 8, tok = blockIdx.x / 8;
  for (uint32_t j = threadIdx.x; j < R / 64; j += 256)
    glu_finish8<S>(part, splits, R, batch, y, xs, act, dn, tok, (x + 8 * (j / 16)) * 128 + (j % 16) * 8);
}

static bool qgemm_supported(const Matrix &w) {
  if (w.layout != LAYOUT_PLANAR) return false;
  if (w.type == Q4_K || w.type == Q5_K || w.type == Q6_K) return w.cols % 256 == 0;
  return (w.type == Q8_0 || w.type == Q4_0) && w.cols % QG_K == 0;
}

// The type pairs (t0 <= t1) with a grouped kernel: every type alone, and the mixes of real
// checkpoints (K-quant projections beside Q6_K or Q8_0 ones).
static bool qgemm_pair(int a, int b) {
  if (a == b) return true;
  return (a == Q4_K && b == Q6_K) || (a == Q8_0 && b == Q4_K) || (a == Q8_0 && b == Q6_K) ||
         (a == Q4_K && b == Q5_K) || (a == Q5_K && b == Q6_K);
}

// The launch's two weight types (t[0] <= t[1]); false for more than two.
static bool group_types(const GemmGroup &g, int t[2]) {
  t[0] = t[1] = -1;
  for (uint32_t j = 0; j < g.n; j++) {
    const int ty = g.job[j].w->type;
    if (ty == t[0] || ty == t[1]) continue;
    if (t[0] < 0) t[0] = ty;
    else if (t[1] < 0) t[1] = ty;
    else return false;
  }
  if (t[1] < 0) t[1] = t[0];
  if (t[0] > t[1]) std::swap(t[0], t[1]);
  return true;
}

bool gemm_group_ok(const GemmGroup &g, uint32_t batch) {
  if (!g.n || g.n > QG_MAX_JOBS || !batch) return false;
  for (uint32_t j = 0; j < g.n; j++)
    if (!g.job[j].w || !g.job[j].w->data || !qgemm_supported(*g.job[j].w) || g.job[j].w->cols != g.job[0].w->cols)
      return false;
  if (g.glu_out && (g.n != 2 || g.job[0].w->rows != g.job[1].w->rows || g.job[0].w->rows % QG_K)) return false;
  int t[2];
  return group_types(g, t) && qgemm_pair(t[0], t[1]);
}

// K span per workgroup: enough splits for two workgroups per CU, each
// at least one 256-column block (64 columns when every matrix is Q8_0), and no more partial
// sums than the scratch holds.
static uint32_t group_kspan(const GemmGroup &g, uint32_t batch, uint64_t scratch_floats, uint32_t *rows_total) {
  // splits end on K tiles (each chunk reads its own block's header, so a split may start
  // inside a 256-column super-block): finer splits fill the chip closer to its target
  const uint32_t align = QG_K;
  uint32_t tiles = 0, rows = 0;
  for (uint32_t j = 0; j < g.n; j++) {
    const Matrix &w = *g.job[j].w;
    tiles += (w.rows + QG_M - 1) / QG_M;
    rows += w.rows;
  }
  tiles *= (batch + QG_N - 1) / QG_N;
  *rows_total = rows;
  const uint32_t cols = g.job[0].w->cols, target = 2 * (uint32_t)device_cu_count();
  uint32_t splits = tiles >= target ? 1 : target / tiles;
  const uint32_t units = cols / align;
  if (splits > units) splits = units;
  if (splits > 16) splits = 16;
  // The workgroups run in rounds of `target` slots, and a short last round leaves CUs idle
  // (336 gate/up tiles in one split fill 66% of one round). Up to twice the splits are
  // considered, and one that fills its rounds at least 10 points better is taken: 336 tiles
  // then run in 3 splits, 1008 workgroups in two rounds at 98%. The split count is
  // ceil(units / per) for the span per = ceil(units / s).
  auto workgroups = [&](uint32_t s) {
    const uint32_t per = (units + s - 1) / s;
    return (uint64_t)tiles * ((units + per - 1) / per);
  };
  auto rounds = [&](uint64_t wg) { return (wg + target - 1) / target; };
  uint64_t bw = workgroups(splits);
  const uint32_t s0 = splits;
  for (uint32_t s = s0 + 1; s <= 2 * s0 + 1 && s <= units && s <= 16; s++) {
    const uint64_t w = workgroups(s);
    // w / (rounds(w) T) > bw / (rounds(bw) T) + 0.1, times 10 rounds(w) rounds(bw) T
    if (10 * w * rounds(bw) > 10 * bw * rounds(w) + rounds(w) * rounds(bw) * target) { splits = s; bw = w; }
  }
  while (splits > 1 && (uint64_t)splits * batch * rows > scratch_floats) splits--;
  const uint32_t per = (units + splits - 1) / splits;
  return per * align;
}

uint64_t gemm_group_split_floats(const GemmGroup &g, uint32_t batch) {
  if (!gemm_group_ok(g, batch)) return 0;
  uint32_t rows = 0;
  const uint32_t kspan = group_kspan(g, batch, ~0ull, &rows);
  const uint32_t splits = (g.job[0].w->cols + kspan - 1) / kspan;
  // the GLU finish and a kept group read their partials whole, so they always have room
  return splits > 1 || g.glu_out || g.keep_partials ? (uint64_t)splits * batch * rows : 0;
}

uint64_t gemm_split_floats(const Matrix &w, uint32_t batch) {
  GemmGroup g;
  g.job[0].w = &w; g.n = 1;
  return gemm_group_split_floats(g, batch);
}

uint64_t gemm_input_elems(uint32_t cols, uint32_t batch) {
  return (uint64_t)(batch + QG_N - 1) / QG_N * QG_N * cols * 2;
}

bool gemm_splits_input(const Matrix &w, const GemmScratch *scratch, uint32_t batch) {
  return qgemm_supported(w) && scratch && scratch->xs && scratch->xs_elems >= gemm_input_elems(w.cols, batch);
}

template <int T0, int T1>
static void launch_qgemm(hipStream_t s, dim3 grid, const QGemm &q) {
  lds_opt_in((const void *)k_gemm_q<T0, T1>);
  hipLaunchKernelGGL((k_gemm_q<T0, T1>), grid, dim3(256), QG_LDS, s, q);
}

hipError_t gemm_group(hipStream_t s, const GemmGroup &g, const float *x, uint32_t batch, GemmScratch *scratch) {
  if (!batch) return hipSuccess;
  const uint32_t cols = g.job[0].w->cols;
  if (!gemm_group_ok(g, batch) || !scratch || !scratch->xs || scratch->xs_elems < gemm_input_elems(cols, batch) ||
      (uintptr_t)x % 16)
    return hipErrorInvalidValue;
  if (g.glu_out && (scratch->xs_elems < gemm_input_elems(g.job[0].w->rows, batch) || (uintptr_t)g.glu_out % 16))
    return hipErrorInvalidValue;
  if (scratch->xs_of != x || scratch->xs_cols != cols || scratch->xs_batch != batch) {
    const uint32_t count = (uint32_t)(gemm_input_elems(cols, batch) / 16);
    hipLaunchKernelGGL(k_gemm_split, dim3((count + 255) / 256), dim3(256), 0, s, x, scratch->xs, cols, batch, count);
    WGD_HIP(hipGetLastError());
    scratch->xs_of = x; scratch->xs_cols = cols; scratch->xs_batch = batch;
  }
  int types[2];
  group_types(g, types);
  QGemm q{};
  q.njobs = g.n; q.xs = scratch->xs; q.cols = cols; q.batch = batch; q.accumulate = g.accumulate ? 1u : 0u;
  uint32_t tiles = 0, row0 = 0;
  for (uint32_t j = 0; j < g.n; j++) {
    const Matrix &w = *g.job[j].w;
    const uint64_t wbytes = planar_bytes(w.type, w.cols, w.rows);
    if (wbytes >= (1ull << 31)) return hipErrorInvalidValue;
    QJob &jb = q.job[j];
    jb.w = w.data; jb.wbytes = (uint32_t)wbytes;
    jb.C = w.cols / chunk_elems(w.type); jb.bpr = w.cols / block_size(w.type); jb.nbp = jb.bpr * (uint32_t)tile_rows(w.rows);
    jb.rows = w.rows; jb.tiles = (w.rows + QG_M - 1) / QG_M; jb.kind = w.type == types[0] ? 0u : 1u; jb.row0 = row0;
    jb.y = g.job[j].y; jb.stride = g.job[j].stride; jb.row_base = g.job[j].row_base;
    tiles += jb.tiles; row0 += w.rows;
  }
  q.kspan = group_kspan(g, batch, scratch->p ? scratch->floats : 0, &q.rows_total);
  const uint32_t splits = (cols + q.kspan - 1) / q.kspan;
  // the GLU finish and a kept group always reduce from the partials (a single split too)
  const bool partials = splits > 1 || g.glu_out || g.keep_partials;
  if (partials && (!scratch->p || (uint64_t)splits * batch * q.rows_total > scratch->floats)) return hipErrorInvalidValue;
  // the finishes read the partials through 32-bit buffer offsets
  if (partials && (splits > MAX_SPLITS || (uint64_t)splits * batch * q.rows_total * 4 >= (1ull << 31)))
    return hipErrorInvalidValue;
  q.part = partials ? scratch->p : nullptr;
  const dim3 grid(tiles, (batch + QG_N - 1) / QG_N, splits);
  const int a = types[0], b = types[1];
  if (a == Q4_K && b == Q4_K) launch_qgemm<Q4_K, Q4_K>(s, grid, q);
  else if (a == Q6_K && b == Q6_K) launch_qgemm<Q6_K, Q6_K>(s, grid, q);
  else if (a == Q8_0 && b == Q8_0) launch_qgemm<Q8_0, Q8_0>(s, grid, q);
  else if (a == Q4_K && b == Q6_K) launch_qgemm<Q4_K, Q6_K>(s, grid, q);
  else if (a == Q8_0 && b == Q4_K) launch_qgemm<Q8_0, Q4_K>(s, grid, q);
  else if (a == Q8_0 && b == Q6_K) launch_qgemm<Q8_0, Q6_K>(s, grid, q);
  else if (a == Q5_K && b == Q5_K) launch_qgemm<Q5_K, Q5_K>(s, grid, q);
  else if (a == Q4_0 && b == Q4_0) launch_qgemm<Q4_0, Q4_0>(s, grid, q);
  else if (a == Q4_K && b == Q5_K) launch_qgemm<Q4_K, Q5_K>(s, grid, q);
  else if (a == Q5_K && b == Q6_K) launch_qgemm<Q5_K, Q6_K>(s, grid, q);
  else return hipErrorInvalidValue;
  WGD_HIP(hipGetLastError());
  if (g.glu_out) {
    const uint32_t R = g.job[0].w->rows, count = batch * (R / 8);
    const uint32_t by_xcd = R % 1024 == 0 && tiles % 8 == 0 ? 1u : 0u;
    const dim3 grid(by_xcd ? batch * 8 : (count + 255) / 256);
    const float *part = q.part;
    float *y = g.glu_f32 ? g.glu_out : nullptr;
    if (splits <= 2)
      hipLaunchKernelGGL(k_glu_reduce<2>, grid, dim3(256), 0, s, part, splits, R, batch, y, scratch->xs, g.glu_act,
                         g.glu_norm, by_xcd);
    else if (splits <= 4)
      hipLaunchKernelGGL(k_glu_reduce<4>, grid, dim3(256), 0, s, part, splits, R, batch, y, scratch->xs, g.glu_act,
                         g.glu_norm, by_xcd);
    else
      hipLaunchKernelGGL(k_glu_reduce<MAX_SPLITS>, grid, dim3(256), 0, s, part, splits, R, batch, y, scratch->xs,
                         g.glu_act, g.glu_norm, by_xcd);
    WGD_HIP(hipGetLastError());
    scratch->xs_of = g.glu_out; scratch->xs_cols = R; scratch->xs_batch = batch;
  } else if (g.keep_partials) {
    if (g.splits) *g.splits = splits;
  } else if (splits > 1) {
    const uint64_t n = (uint64_t)q.rows_total * batch;
    uint32_t blocks = (uint32_t)((n + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    if (splits <= 4) hipLaunchKernelGGL(k_gemm_reduce<4>, dim3(blocks), dim3(256), 0, s, q, splits);
    else hipLaunchKernelGGL(k_gemm_reduce<MAX_SPLITS>, dim3(blocks), dim3(256), 0, s, q, splits);
  }
  return hipGetLastError();
}

hipError_t gemm(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                uint32_t row_base, uint32_t input_offset, uint32_t batch, GemmScratch *scratch, bool accumulate) {
  if (!w.rows || !batch) return hipSuccess;
  const float *xb = x + (uint64_t)input_offset * w.cols;
  if (gemm_splits_input(w, scratch, batch) && (uintptr_t)xb % 16 == 0) {
    GemmGroup g;
    g.job[0] = GemmJob{&w, y, stride, row_base};
    g.n = 1; g.accumulate = accumulate;
    return gemm_group(s, g, xb, batch, scratch);
  }
  if (accumulate) return hipErrorInvalidValue;  // only the planar-weight GEMM adds into y
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
