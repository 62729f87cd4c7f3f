// decode.h — device-side GGUF element decode and wavefront reductions shared by the
// kernels of libwgd (header-only so every translation unit inlines them).
#pragma once
#include "internal.h"

namespace wgd {

__device__ __forceinline__ uint32_t block_size_dev(int t) { return t == Q6_K || t == Q4_K || t == Q5_K ? 256u : (t == Q8_0 || t == Q4_0 ? 32u : 1u); }

// ------------------------------------------------------------------ exact decode

// IEEE half -> float from the bit fields (quant.ts:2-5); exact for subnormals.
__device__ __forceinline__ float half_bits(uint32_t h) {
  uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 31u, f = h & 1023u;
  if (e == 0) { float v = (float)f * 5.9604644775390625e-8f; return sign ? -v : v; }
  if (e == 31) return __uint_as_float(sign | 0x7f800000u | (f << 13));
  return __uint_as_float(sign | ((e + 112u) << 23) | (f << 13));
}
__device__ __forceinline__ uint32_t byte_at(const uint8_t *b, uint64_t p) { return b[p]; }
__device__ __forceinline__ float f16_at(const uint8_t *b, uint64_t p) {
  return half_bits(b[p] | ((uint32_t)b[p + 1] << 8));
}

// One element of a GGUF tensor, evaluated in f32 in the reference's operation order.
__device__ __forceinline__ float deq_elem(int type, const uint8_t *b, uint64_t i) {
  switch (type) {
    case F32: return __uint_as_float(b[4 * i] | (b[4 * i + 1] << 8) | (b[4 * i + 2] << 16) | ((uint32_t)b[4 * i + 3] << 24));
    case F16: return f16_at(b, 2 * i);
    case Q4_0: {
      uint64_t p = (i / 32) * 18; uint32_t j = i % 32;
      return f16_at(b, p) * (float)((int)((byte_at(b, p + 2 + j % 16) >> ((j / 16) * 4)) & 15u) - 8);
    }
    case Q8_0: {
      uint64_t p = (i / 32) * 34;
      return f16_at(b, p) * (float)(int8_t)byte_at(b, p + 2 + i % 32);
    }
    case Q4_K: case Q5_K: {
      uint64_t p = (i / 256) * (type == Q4_K ? 144 : 176); uint32_t j = i % 256, s = j / 32;
      uint32_t sc, mn;
      if (s < 4) { sc = byte_at(b, p + 4 + s) & 63u; mn = byte_at(b, p + 8 + s) & 63u; }
      else {
        sc = (byte_at(b, p + 8 + s) & 15u) | ((byte_at(b, p + s) >> 6) << 4);
        mn = (byte_at(b, p + 8 + s) >> 4) | ((byte_at(b, p + 4 + s) >> 6) << 4);
      }
      uint32_t q = (byte_at(b, p + (type == Q4_K ? 16 : 48) + (j / 64) * 32 + j % 32) >> ((s % 2) * 4)) & 15u;
      if (type == Q5_K) q |= ((byte_at(b, p + 16 + j % 32) >> s) & 1u) << 4;
      return f16_at(b, p) * (float)(sc * q) - f16_at(b, p + 2) * (float)mn;
    }
    case Q6_K: {
      uint64_t p = (i / 256) * 210; uint32_t j = i % 256, seg = j / 128, qtr = (j % 128) / 32, ln = j % 32;
      uint32_t lo = (byte_at(b, p + seg * 64 + (qtr % 2) * 32 + ln) >> ((qtr / 2) * 4)) & 15u;
      uint32_t hi = (byte_at(b, p + 128 + seg * 32 + ln) >> (qtr * 2)) & 3u;
      float sc = (float)(int8_t)byte_at(b, p + 192 + seg * 8 + qtr * 2 + ln / 16);
      return f16_at(b, p + 208) * sc * (float)((int)(lo | (hi << 4)) - 32);
    }
  }
  return __uint_as_float(0x7fc00000u);
}

// ------------------------------------------------------------------ planar chunk layouts
// (written by repack_planar, quant.hip): chunk (row, c) of 32 elements in a tiled plane.

// Q4_K quant of element k of `row` (C chunks per row): chunk k / 32, byte k % 16, nibble (k % 32) / 16.
__device__ __forceinline__ uint32_t q4_quant(const uint8_t *w, uint32_t row, uint32_t C, uint32_t k) {
  const uint32_t e = k % 32;
  return (w[tiled(row, k / 32, C) * 16 + (e & 15)] >> (4 * (e >> 4))) & 15u;
}
// Q6_K 6-bit quant of element k: low nibble as Q4_K in the ql plane; the high 2 bits of chunk
// element e in qh byte 4 * ((e % 16) / 8) + e % 4 at bit 4 * ((e % 8) / 4) + 2 * (e / 16).
__device__ __forceinline__ uint32_t q6_quant(const uint8_t *w, uint64_t nbp, uint32_t row, uint32_t C, uint32_t k) {
  const Q6Planes p = q6_planes(nbp);
  const uint32_t e = k % 32;
  const uint64_t ci = tiled(row, k / 32, C);
  const uint32_t lo = (w[p.ql + ci * 16 + (e & 15)] >> (4 * (e >> 4))) & 15u;
  const uint32_t r = e & 15;
  const uint32_t hi = (w[p.qh + ci * 8 + 4 * (r >> 3) + (r & 3)] >> (4 * ((r & 7) >> 2) + 2 * (e >> 4))) & 3u;
  return lo | (hi << 4);
}

// ------------------------------------------------------------------ wave reduction

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over aligned segments of `width` lanes (16, 32 or 64) with DPP moves, which stay in
// the VALU (no LDS crossbar round trip per step): quad xor 1, quad xor 2, half-row mirror and
// row mirror leave each 16-lane row's sum in all of its lanes; row_bcast15 / row_bcast31
// fold rows into rows 1, 3 and then 3. The segment sum ends in its last lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float seg_sum(float v, uint32_t width) {
  v = dpp_add<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror
  if (width >= 32) v = dpp_add<0x142, 0xa>(v);  // row_bcast15 into rows 1 and 3
  if (width == 64) v = dpp_add<0x143, 0xc>(v);  // row_bcast31 into rows 2 and 3
  return v;
}

// Wave-wide sum, the same value returned in every lane (DPP folds into lane 63, then a
// scalar read).
__device__ __forceinline__ float wave_total(float v) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(seg_sum(v, 64)), 63));
}

// Sum within aligned segments of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float segment_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ------------------------------------------------------------------ split-K partial sums
// The split-K GEMMs leave partial sums part[z][...] for z < splits (at most MAX_SPLITS),
// `stride` floats apart. These add one element's (or four consecutive elements') partials
// in split order, the adds of a loop over z, with every split's load issued before the
// first add: raw buffer loads over the partial buffer (4 * splits * stride bytes, below
// 2^31), so the loads of the splits past `splits` read zero without touching memory, and
// selects leave them out of the sum.
constexpr uint32_t MAX_SPLITS = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t split_rsrc(const float *part, uint32_t splits, uint64_t stride) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(part), (short)0, (int)(4 * splits * stride), 0x00020000);
}
// Elements at byte offset `off` of split 0; splits are `sb` bytes apart.
template <uint32_t S>
__device__ __forceinline__ float split_sum(__amdgpu_buffer_rsrc_t r, uint32_t splits, uint32_t sb, uint32_t off) {
  float p[S];
#pragma unroll
  for (uint32_t z = 0; z < S; z++) p[z] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off + z * sb, 0, 0));
  float a = 0.f;
#pragma unroll
  for (uint32_t z = 0; z < S; z++) a = z < splits ? a + p[z] : a;
  return a;
}
template <uint32_t S>
__device__ __forceinline__ float4 split_sum4(__amdgpu_buffer_rsrc_t r, uint32_t splits, uint32_t sb, uint32_t off) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  u4 p[S];
#pragma unroll
  for (uint32_t z = 0; z < S; z++) p[z] = __builtin_amdgcn_raw_buffer_load_b128(r, off + z * sb, 0, 0);
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (uint32_t z = 0; z < S; z++) {
    const bool in = z < splits;
    a.x = in ? a.x + __uint_as_float(p[z].x) : a.x;
    a.y = in ? a.y + __uint_as_float(p[z].y) : a.y;
    a.z = in ? a.z + __uint_as_float(p[z].z) : a.z;
    a.w = in ? a.w + __uint_as_float(p[z].w) : a.w;
  }
  return a;
}

// ------------------------------------------------------------------ argmax keys
// Key = (order-preserving bits of the value) << 32 | (~index): the largest key is the
// largest finite value with the lowest index. Non-finite entries never produce a key, so
// key 0 means "no finite logit".
__device__ __forceinline__ uint64_t arg_key(float f, uint32_t i) {
  if (!isfinite(f)) return 0;
  uint32_t u = f == 0.f ? 0u : __float_as_uint(f);
  uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - i);
}
__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)k, o, 64), hi = __shfl_xor((uint32_t)(k >> 32), o, 64);
    k = key_max(k, ((uint64_t)hi << 32) | lo);
  }
  return k;
}

}  // namespace wgd
