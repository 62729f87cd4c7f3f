// split.h — the prompt GEMM's activation format: bf16 (hi, lo) pairs in MFMA fragment order.
//
// bf16 keeps 8 significant bits, so a value is carried as v = hi + lo with hi = RN_bf16(v)
// and lo = RN_bf16(v - hi) (about 16 bits together). The activations [batch][cols] are
// stored as 128-token x 64-column tiles, tile (n, k) at (n * cols / 64 + k) * SPLIT_TILE
// bf16. Inside a tile, [hl][b][s][g][c][e] holds token 16 b + c, column 32 s + 8 g + e of
// the hi (hl = 0) or lo (hl = 1) part: lane 16 g + c of a v_mfma_f32_16x16x32_bf16 takes
// the 16 bytes at fragment (hl, b, s) + 16 * lane. Producers that already hold a batch of
// activations (RMSNorm, the GLU) write this form beside their f32 output so the GEMMs that
// read it need no split pass of their own.
#pragma once
#include "internal.h"

namespace wgd {

constexpr uint32_t SPLIT_N = 128, SPLIT_K = 64;
constexpr uint32_t SPLIT_FRAG = 512;                     // bf16 of one 16 x 32 fragment
constexpr uint32_t SPLIT_TILE = 2 * 8 * 2 * SPLIT_FRAG;  // bf16 of a 128 x 64 tile, hi and lo

__host__ __device__ constexpr uint32_t frag_at(uint32_t hl, uint32_t b, uint32_t s, uint32_t g, uint32_t c) {
  return ((((hl * 8 + b) * 2 + s) * 4 + g) * 16 + c) * 8;
}

#ifdef __HIPCC__
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> (hi, lo) bf16 pairs with hi = RN(v), lo = RN(v - hi) (native gfx950 packing).
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
  const f32x2 v = {a, b};
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  const f32x2 back = {__uint_as_float(hi << 16), __uint_as_float(hi & 0xFFFF0000u)};
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(v - back, bf16x2));
}

// The gate activations of the GLU: SiLU (act 0) and tanh-approximated GELU (act 1).
__device__ __forceinline__ float glu_act(float x, int act) {
  if (!act) return x / (1.f + expf(-x));
  return 0.5f * x * (1.f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}

// Columns k..k+7 (k % 8 == 0) of token tok.
__device__ __forceinline__ void split_store8(uint16_t *xs, uint32_t cols, uint32_t tok, uint32_t k, float4 a, float4 b) {
  uint32_t h[4], l[4];
  split2(a.x, a.y, h[0], l[0]);
  split2(a.z, a.w, h[1], l[1]);
  split2(b.x, b.y, h[2], l[2]);
  split2(b.z, b.w, h[3], l[3]);
  const uint32_t r = tok % SPLIT_N, kk = k % SPLIT_K;
  uint16_t *t = xs + ((uint64_t)(tok / SPLIT_N) * (cols / SPLIT_K) + k / SPLIT_K) * SPLIT_TILE;
  *(uint4 *)(t + frag_at(0, r / 16, kk / 32, (kk % 32) / 8, r % 16)) = make_uint4(h[0], h[1], h[2], h[3]);
  *(uint4 *)(t + frag_at(1, r / 16, kk / 32, (kk % 32) / 8, r % 16)) = make_uint4(l[0], l[1], l[2], l[3]);
}
#endif

}  // namespace wgd
