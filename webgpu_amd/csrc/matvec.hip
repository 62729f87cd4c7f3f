// matvec.hip — decode dequant-matvec (batch 1) for gfx950 on int8 matrix cores.
//
// Replaces matmulShader (src/core/shaders.ts:39-54) for one activation row. The reference
// decodes every weight to f32 and multiplies by an f32 activation. Here the activation row
// is quantized first ("QX" format): per 16-element block a scale s = max|x| / 127 and three
// signed base-254 digits per element, x = s * (d0 + d1/254 + d2/254^2) (error <= 6.1e-8 *
// max|x|, f32-level). Weights stay in their raw form: 4-bit (Q4_K), 6-bit (Q6_K) or 8-bit
// (Q8_0) quants, and 5-bit (Q5_K) and 4-bit offset (Q4_0) ones, become int8 operands of v_mfma_i32_16x16x64_i8, whose int32 sums are exact.
// Block scales apply once per 16 elements; the Q4_K minimum and the Q6_K offset use the
// exact sums of x.
//
// MFMA mapping (D = A x B, 16 x 16 x 64): B holds weights, column = row r of W (lane
// r % 16), K-group g = lane / 16 = 16 quants of chunk column 4q + g; A is the activation
// digits, block-diagonal: A row 4g + p holds digit p of the K-group g elements (p < 3,
// zero elsewhere). D lane (r, g) then holds the three digit sums of its own row and chunk,
// so digit combination, the block scales and the Q4_K scale/min (from the header the same
// lane loaded) are applied in-lane with no cross-lane traffic. A 16-byte chunk (32
// elements) feeds two MFMAs (low and high nibbles); a Q8_0 chunk (16 elements) one.
//
// Memory: planar row-tiled weights (quant.hip): one load instruction of a wavefront reads 16
// rows x 4 chunks = 1 KB contiguous; raw buffer loads with the per-unit offset in an SGPR.
// Each wavefront keeps DU units of loads in flight (software pipeline over registers). The
// activation digits are staged once per workgroup in LDS: their loads are issued before the
// first weight loads (loads complete in order, so a later issue would wait on every weight
// load in flight) and written to LDS once they arrive. Per row step each lane leaves its partial sum in LDS; the first RT threads add the
// K slices and column groups in a fixed order (deterministic) and run the epilogue: store,
// residual add, or the gated SwiGLU/GeGLU of a gate/up pair, optionally re-quantizing the
// result (times the next RMSNorm weight) for the next matvec. Nothing synchronizes across
// workgroups inside a launch: on MI355X each XCD has its own L2, and device-scope fences
// write back and invalidate it.
#include <chrono>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <utility>
#include <vector>

#include "internal.h"
#include "decode.h"
#include "matvec.h"

namespace wgd {

// ------------------------------------------------------------------ quantization helpers

// Standalone quantization of x (length K), optionally as x * w: one workgroup per 256.
__global__ __launch_bounds__(256) void k_quantize(const float *x, uint32_t K, const float *w, QXOut q) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  const bool live = i < K;
  const float v = live ? x[i] : 0.f;
  qx_store(q, i, (live && w) ? v * w[i] : v, v, live);
}

// ------------------------------------------------------------------ chunk kernels

typedef int v4i __attribute__((ext_vector_type(4)));

// Weight loads: raw buffer loads over the matrix allocation (a 128-bit resource in SGPRs),
// per-lane offset in a VGPR, per-unit offset in an SGPR; offsets past the allocation read
// zero. Non-temporal: weight bytes are read once per token.
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
constexpr int CPOL_NT = 2;
__device__ __forceinline__ Rsrc make_rsrc(const uint8_t *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bl16(Rsrc r, uint32_t v, uint32_t s) {
  const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(r, v, s, CPOL_NT);
  return make_uint4(x.x, x.y, x.z, x.w);
}
__device__ __forceinline__ uint2 bl8(Rsrc r, uint32_t v, uint32_t s) {
  const u32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(r, v, s, CPOL_NT);
  return make_uint2(x.x, x.y);
}
__device__ __forceinline__ uint32_t bl4(Rsrc r, uint32_t v, uint32_t s) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, v, s, CPOL_NT);
}
__device__ __forceinline__ uint32_t bl2(Rsrc r, uint32_t v, uint32_t s) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, v, s, CPOL_NT);
}
// Activation loads: cached (every workgroup reads the same vector), zero past the plane.
__device__ __forceinline__ uint4 bl16c(Rsrc r, uint32_t v) {
  const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(r, v, 0, 0);
  return make_uint4(x.x, x.y, x.z, x.w);
}
__device__ __forceinline__ uint32_t bl4c(Rsrc r, uint32_t v) { return __builtin_amdgcn_raw_buffer_load_b32(r, v, 0, 0); }
__device__ __forceinline__ float f16lo(uint32_t v) { return __half2float(__ushort_as_half((unsigned short)(v & 0xFFFFu))); }

__device__ __forceinline__ float f16hi(uint32_t v) { return __half2float(__ushort_as_half((unsigned short)(v >> 16))); }
__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, v4i{0, 0, 0, 0}, 0, 0, 0);
}

// Digit sums of one MFMA output lane -> f32: s0 * 254^2 + s1 * 254 + s2. For 4-bit weights
// the weighted sum is exact in int32 (|s0| <= 16 * 15 * 127); wider weights form the first
// two digits in integers and the last step in f32.
__device__ __forceinline__ float dig4(v4i d) { return (float)(__mul24(d[0], 64516) + __mul24(d[1], 254) + d[2]); }
__device__ __forceinline__ float dig8(v4i d) { return fmaf((float)(__mul24(d[0], 254) + d[1]), 254.f, (float)d[2]); }

// One unit: tile T (16 rows) and the first of its 8 chunk columns (cb % 8 == 0). A lane
// (row r, group g) takes columns cb + g and cb + 4 + g: for the K-quants the two sub-blocks
// g and 4 + g of one 256-element block, so its scale fields are at lane-constant bit offsets.
struct Unit { uint32_t T, cb; };

// Activation of a lane's two chunk columns, read from LDS: per column the A operands of its
// 16-element K-groups (block-diagonal digits) and, per 16 elements, the block scale (divided
// by 254^2) and the exact block sum.
struct XA { v4i a[2][2]; float s[2][2], m[2][2]; };

constexpr uint32_t M4 = 0x0F0F0F0Fu;

// Q4_K: chunk byte i = q[i] | q[i + 16] << 4; header plane: the GGUF header (d, dmin, 12
// bytes of packed 6-bit scales/mins, quant.ts:10-16). Sub-block g: scale and min are the
// low 6 bits of header bytes 4 + g and 8 + g; sub-block 4 + g: low 4 bits of byte 12 + g
// (scale) and its high 4 bits (min), top 2 bits from bytes 4 + g and 8 + g.
struct CQ4K {
  static constexpr int N = 32;
  struct W { uint4 q0, q1, h; };
  struct L { uint32_t vq, vh, g8; };
  static __device__ __forceinline__ L lane(uint32_t r, uint32_t g) { return L{256 * g + 16 * r, 16 * r, 8 * g}; }
  static __device__ __forceinline__ W load(Rsrc w, const MVSeg &s, uint32_t C, const Unit &u, const L &l) {
    W r;
    const uint32_t so = 256 * (u.T * C + u.cb);
    r.q0 = bl16(w, l.vq, so);
    r.q1 = bl16(w, l.vq + 1024, so);
    r.h = bl16(w, l.vh, s.nbp * 128 + 256 * (u.T * s.bpr + u.cb / 8));
    return r;
  }
  static __device__ __forceinline__ float chunk(const uint4 &q, const v4i (&a)[2], const float (&sx)[2]) {
    const v4i lo = {(int)(q.x & M4), (int)(q.y & M4), (int)(q.z & M4), (int)(q.w & M4)};
    const v4i hi = {(int)((q.x >> 4) & M4), (int)((q.y >> 4) & M4), (int)((q.z >> 4) & M4), (int)((q.w >> 4) & M4)};
    return fmaf(sx[1], dig4(mfma_i8(a[1], hi)), sx[0] * dig4(mfma_i8(a[0], lo)));
  }
  static __device__ __forceinline__ float dot(const W &r, const L &l, const XA &x) {
    const float ca = chunk(r.q0, x.a[0], x.s[0]), cb = chunk(r.q1, x.a[1], x.s[1]);
    const uint32_t sca = __builtin_amdgcn_ubfe(r.h.y, l.g8, 6), mna = __builtin_amdgcn_ubfe(r.h.z, l.g8, 6);
    const uint32_t scb = __builtin_amdgcn_ubfe(r.h.w, l.g8, 4) | (__builtin_amdgcn_ubfe(r.h.y, l.g8 + 6, 2) << 4);
    const uint32_t mnb = __builtin_amdgcn_ubfe(r.h.w, l.g8 + 4, 4) | (__builtin_amdgcn_ubfe(r.h.z, l.g8 + 6, 2) << 4);
    const float u = fmaf((float)scb, cb, (float)sca * ca);
    const float v = fmaf((float)mnb, x.m[1][0] + x.m[1][1], (float)mna * (x.m[0][0] + x.m[0][1]));
    return fmaf(f16lo(r.h.x), u, -f16hi(r.h.x) * v);
  }
};

// Q6_K: ql byte i = lo4[i] | lo4[i + 16] << 4; qh dword m byte b holds the high 2 bits of
// elements 8m+b, 16+8m+b, 8m+4+b, 16+8m+4+b at bits 0, 2, 4, 6; two int8 scales per chunk
// (one per 16 elements) and the block's f16 d in their planes (quant.ts:21-27).
struct CQ6K {
  static constexpr int N = 32;
  struct W { uint4 q0, q1; uint2 h0, h1; uint32_t s0, s1, d; };
  struct L { uint32_t vq, vh, vs, vd; };
  static __device__ __forceinline__ L lane(uint32_t r, uint32_t g) { return L{256 * g + 16 * r, 128 * g + 8 * r, 32 * g + 2 * r, 2 * r}; }
  static __device__ __forceinline__ W load(Rsrc w, const MVSeg &s, uint32_t C, const Unit &u, const L &l) {
    W r;
    const uint32_t tc = u.T * C + u.cb;
    r.q0 = bl16(w, l.vq, 256 * tc);
    r.q1 = bl16(w, l.vq + 1024, 256 * tc);
    r.h0 = bl8(w, l.vh, s.nbp * 128 + 128 * tc);
    r.h1 = bl8(w, l.vh + 512, s.nbp * 128 + 128 * tc);
    r.s0 = bl2(w, l.vs, s.nbp * 192 + 32 * tc);
    r.s1 = bl2(w, l.vs + 128, s.nbp * 192 + 32 * tc);
    r.d = bl2(w, l.vd, s.nbp * 208 + 32 * (u.T * s.bpr + u.cb / 8));
    return r;
  }
  static __device__ __forceinline__ float chunk(const uint4 &qq, const uint2 &h, uint32_t sc, const v4i (&a)[2],
                                                const float (&sx)[2], const float (&mx)[2]) {
    const uint32_t q[4] = {qq.x, qq.y, qq.z, qq.w};
    v4i blo, bhi;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t Q = (k < 2 ? h.x : h.y) >> (4 * (k & 1));
      blo[k] = (int)((q[k] & M4) | ((Q << 4) & 0x30303030u));
      bhi[k] = (int)(((q[k] >> 4) & M4) | ((Q << 2) & 0x30303030u));
    }
    const float cl = dig8(mfma_i8(a[0], blo)), ch = dig8(mfma_i8(a[1], bhi));
    const float s0 = (float)(int8_t)(sc & 0xFFu), s1 = (float)(int8_t)((sc >> 8) & 0xFFu);
    return fmaf(s1, fmaf(sx[1], ch, -32.f * mx[1]), s0 * fmaf(sx[0], cl, -32.f * mx[0]));
  }
  static __device__ __forceinline__ float dot(const W &r, const L &, const XA &x) {
    return f16lo(r.d) * (chunk(r.q0, r.h0, r.s0, x.a[0], x.s[0], x.m[0]) + chunk(r.q1, r.h1, r.s1, x.a[1], x.s[1], x.m[1]));
  }
};

// Q8_0: a chunk is half a block, 16 int8 quants (already MFMA operands); d per block
// (quant.ts:8). A unit is four blocks per row; a lane's columns cb + g and cb + 4 + g are in
// blocks cb / 2 + g / 2 and two after it.
struct CQ80 {
  static constexpr int N = 16;
  struct W { uint4 q0, q1; uint32_t d0, d1; };
  struct L { uint32_t vq, vd; };
  static __device__ __forceinline__ L lane(uint32_t r, uint32_t g) { return L{256 * g + 16 * r, 32 * (g >> 1) + 2 * r}; }
  static __device__ __forceinline__ W load(Rsrc w, const MVSeg &s, uint32_t C, const Unit &u, const L &l) {
    W r;
    const uint32_t so = 256 * (u.T * C + u.cb), sd = s.nbp * 32 + 32 * (u.T * s.bpr + u.cb / 2);
    r.q0 = bl16(w, l.vq, so);
    r.q1 = bl16(w, l.vq + 1024, so);
    r.d0 = bl2(w, l.vd, sd);
    r.d1 = bl2(w, l.vd + 64, sd);
    return r;
  }
  static __device__ __forceinline__ float dot(const W &r, const L &, const XA &x) {
    const v4i b0 = {(int)r.q0.x, (int)r.q0.y, (int)r.q0.z, (int)r.q0.w}, b1 = {(int)r.q1.x, (int)r.q1.y, (int)r.q1.z, (int)r.q1.w};
    return fmaf(f16lo(r.d1) * x.s[1][0], dig8(mfma_i8(x.a[1][0], b1)), f16lo(r.d0) * x.s[0][0] * dig8(mfma_i8(x.a[0][0], b0)));
  }
};

// Q5_K: Q4_K with a fifth bit per quant (quant.ts:13-19). The low nibbles and the header
// are laid out as for Q4_K; each chunk's fifth bits are one dword whose byte b holds, at bit
// k, element 4k + b and at bit 4 + k element 16 + 4k + b, so one shift and mask per operand
// dword moves four of them to bit 4 of their bytes. Quants reach 31: the digit sums take
// the f32 last step.
struct CQ5K {
  static constexpr int N = 32;
  struct W { uint4 q0, q1, h; uint32_t b0, b1; };
  struct L { uint32_t vq, vb, vh, g8; };
  static __device__ __forceinline__ L lane(uint32_t r, uint32_t g) { return L{256 * g + 16 * r, 64 * g + 4 * r, 16 * r, 8 * g}; }
  static __device__ __forceinline__ W load(Rsrc w, const MVSeg &s, uint32_t C, const Unit &u, const L &l) {
    W r;
    const uint32_t tc = u.T * C + u.cb;
    r.q0 = bl16(w, l.vq, 256 * tc);
    r.q1 = bl16(w, l.vq + 1024, 256 * tc);
    r.b0 = bl4(w, l.vb, s.nbp * 128 + 64 * tc);
    r.b1 = bl4(w, l.vb + 256, s.nbp * 128 + 64 * tc);
    r.h = bl16(w, l.vh, s.nbp * 160 + 256 * (u.T * s.bpr + u.cb / 8));
    return r;
  }
  static __device__ __forceinline__ float chunk(const uint4 &qq, uint32_t B, const v4i (&a)[2], const float (&sx)[2]) {
    const uint32_t q[4] = {qq.x, qq.y, qq.z, qq.w};
    v4i lo, hi;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      lo[k] = (int)((q[k] & M4) | ((B << (4 - k)) & 0x10101010u));
      hi[k] = (int)(((q[k] >> 4) & M4) | ((B >> k) & 0x10101010u));
    }
    return fmaf(sx[1], dig8(mfma_i8(a[1], hi)), sx[0] * dig8(mfma_i8(a[0], lo)));
  }
  static __device__ __forceinline__ float dot(const W &r, const L &l, const XA &x) {
    const float ca = chunk(r.q0, r.b0, x.a[0], x.s[0]), cb = chunk(r.q1, r.b1, x.a[1], x.s[1]);
    const uint32_t sca = __builtin_amdgcn_ubfe(r.h.y, l.g8, 6), mna = __builtin_amdgcn_ubfe(r.h.z, l.g8, 6);
    const uint32_t scb = __builtin_amdgcn_ubfe(r.h.w, l.g8, 4) | (__builtin_amdgcn_ubfe(r.h.y, l.g8 + 6, 2) << 4);
    const uint32_t mnb = __builtin_amdgcn_ubfe(r.h.w, l.g8 + 4, 4) | (__builtin_amdgcn_ubfe(r.h.z, l.g8 + 6, 2) << 4);
    const float u = fmaf((float)scb, cb, (float)sca * ca);
    const float v = fmaf((float)mnb, x.m[1][0] + x.m[1][1], (float)mna * (x.m[0][0] + x.m[0][1]));
    return fmaf(f16lo(r.h.x), u, -f16hi(r.h.x) * v);
  }
};

// Q4_0: a chunk is a whole block, d * (q - 8) (quant.ts:7); the offset uses the exact
// block sums of x. A lane's chunk columns cb + g and cb + 4 + g are blocks of their own.
struct CQ40 {
  static constexpr int N = 32;
  struct W { uint4 q0, q1; uint32_t d0, d1; };
  struct L { uint32_t vq, vd; };
  static __device__ __forceinline__ L lane(uint32_t r, uint32_t g) { return L{256 * g + 16 * r, 32 * g + 2 * r}; }
  static __device__ __forceinline__ W load(Rsrc w, const MVSeg &s, uint32_t C, const Unit &u, const L &l) {
    W r;
    const uint32_t tc = u.T * C + u.cb;
    r.q0 = bl16(w, l.vq, 256 * tc);
    r.q1 = bl16(w, l.vq + 1024, 256 * tc);
    r.d0 = bl2(w, l.vd, s.nbp * 16 + 32 * tc);
    r.d1 = bl2(w, l.vd + 128, s.nbp * 16 + 32 * tc);
    return r;
  }
  static __device__ __forceinline__ float chunk(const uint4 &q, const v4i (&a)[2], const float (&sx)[2], const float (&mx)[2]) {
    const v4i lo = {(int)(q.x & M4), (int)(q.y & M4), (int)(q.z & M4), (int)(q.w & M4)};
    const v4i hi = {(int)((q.x >> 4) & M4), (int)((q.y >> 4) & M4), (int)((q.z >> 4) & M4), (int)((q.w >> 4) & M4)};
    return fmaf(sx[1], dig4(mfma_i8(a[1], hi)), fmaf(sx[0], dig4(mfma_i8(a[0], lo)), -8.f * (mx[0] + mx[1])));
  }
  static __device__ __forceinline__ float dot(const W &r, const L &, const XA &x) {
    return fmaf(f16lo(r.d1), chunk(r.q1, x.a[1], x.s[1], x.m[1]), f16lo(r.d0) * chunk(r.q0, x.a[0], x.s[0], x.m[0]));
  }
};

// ------------------------------------------------------------------ the tile kernel

__device__ __forceinline__ float gelu_tanh_mv(float g) {
  return 0.5f * g * (1.f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g)));
}

// Per-row inputs of the epilogue (residual, bias, next norm weight), loaded at the start of
// the workgroup so their latency hides behind the weight stream: raw buffer loads that read
// zero past the segment's rows, or for an absent input.
struct RowIn { float y, bias, norm; };
__device__ __forceinline__ RowIn row_inputs(const MV &m, const MVSeg &g, uint32_t row) {
  const uint32_t nb = 4 * g.rows;
  const Rsrc ry = make_rsrc((const uint8_t *)g.y, m.epi == MV_ADD ? nb : 0);
  const Rsrc rb = make_rsrc((const uint8_t *)g.bias, g.bias ? nb : 0);
  const Rsrc rn = make_rsrc((const uint8_t *)m.oq_norm, (m.oq.d0 && m.oq_norm) ? nb : 0);
  RowIn in;
  in.y = __uint_as_float(bl4c(ry, 4 * row));
  in.bias = __uint_as_float(bl4c(rb, 4 * row));
  in.norm = __uint_as_float(bl4c(rn, 4 * row));
  return in;
}

// Epilogue of one row: thread t < RT holds row row0 + t of segment g.
__device__ __forceinline__ float finish_row(const MV &m, const MVSeg &g, uint32_t row, bool live, float v, float u,
                                            const RowIn &in) {
  float out = 0.f;
  if (live) {
    v += in.bias;
    switch (m.epi) {
      case MV_STORE: out = v; break;
      case MV_ADD: out = in.y + v; break;
      case MV_SILU: out = v / (1.f + expf(-v)) * u; break;
      case MV_GELU: out = gelu_tanh_mv(v) * u; break;
    }
    g.y[row] = out;
  }
  if (m.oq.d0) {
    const float wn = (live && m.oq_norm) ? in.norm : 1.f;
    qx_store(m.oq, row, out * wn, out, live);
  }
  return out;
}

// LDS (dynamic): [0, 256) zeros (the A operand reads of off-diagonal lanes) | digit planes p
// at 256 + p * ke | per 16-element block {scale / 254^2, sum} (ke / 16 float pairs) | partial
// sums [NS][RT][4 groups] (two sets for a gated pair) | for an input with a pending RMSNorm,
// the per-block sums of squares (ke / 16 floats).
constexpr uint32_t MV_ZERO = 256;
struct LdsMap { uint32_t digits, sm, vals, vals1, sq, bytes; };
__host__ __device__ inline LdsMap lds_map(uint32_t ke, uint32_t ns, uint32_t rt, bool glu, bool normed) {
  LdsMap l;
  l.digits = MV_ZERO;
  l.sm = MV_ZERO + 3 * ke;
  l.vals = l.sm + 8 * (ke / 16);
  l.vals1 = l.vals + 16 * ns * rt;
  l.sq = l.vals1 + (glu ? 16 * ns * rt : 0);
  l.bytes = l.sq + (normed ? 4 * (ke / 16) : 0);
  return l;
}

// The body of one workgroup: row tile t of segment g, weights of chunk type T.
template <class T, int DU, bool GLU>
__device__ __forceinline__ void mv_tile(const MV &m, const MVSeg &g, uint32_t t, uint8_t *lds) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t s = wv % m.NS, rg = wv / m.NS;
  const LdsMap L = lds_map(m.ke, m.NS, m.RT, GLU, m.x.normed != 0);
  const Rsrc rw = make_rsrc(g.w, g.bytes);
  const Rsrc rw1 = make_rsrc(GLU ? g.w1 : g.w, g.bytes);
  const uint32_t row0 = t * m.RT, tile0 = row0 / 16;
  const uint32_t r = lane & 15, gq = lane >> 4;
  const typename T::L lc = T::lane(r, gq);
  // unit u of this wavefront: step u / NSB (tile tile0 + rg + step * NR), octet (s * NSB + u % NSB)
  // (uniform: readfirstlane keeps the load offsets in SGPRs whatever the divergence analysis
  // concludes about the loop counters)
  auto unit_of = [&](uint32_t step, uint32_t sl) -> Unit {
    return Unit{(uint32_t)__builtin_amdgcn_readfirstlane(tile0 + rg + step * m.NR),
                (uint32_t)__builtin_amdgcn_readfirstlane(8 * (s * m.NSB + sl))};
  };
  typename T::W buf[DU], buf1[GLU ? DU : 1];
  uint32_t is_step = 0, is_sl = 0;  // next unit to issue
  auto issue = [&](int slot) {
    const Unit u = unit_of(is_step, is_sl);
    buf[slot] = T::load(rw, g, m.C, u, lc);
    if (GLU) buf1[slot] = T::load(rw1, g, m.C, u, lc);
    if (++is_sl == m.NSB) { is_sl = 0; is_step++; }
  };
  // The activation is staged in LDS; its loads (from L2) go out first and the first DU units
  // of weight loads right after, so the wait for the activation does not include the weights
  // (loads complete in issue order for the wait counter). The activation loads are raw buffer
  // loads that read zero past each plane, so they need no branches, and nothing uses their
  // values before the weight loads are issued: any arithmetic on them there would make the
  // compiler wait for them first. Up to XJ 16-byte pieces per plane and XB blocks per thread
  // are held in registers; any rest is staged afterwards.
  constexpr uint32_t XJ = 2, XB = 2;
  const uint32_t nt = blockDim.x, tid = threadIdx.x;
  const uint32_t kq = (m.x.len + 63) / 64 * 64;  // QX planes hold Kp elements
  const uint32_t blocks = m.ke / 16, live = m.x.len / 16;
  const Rsrc rxd[3] = {make_rsrc((const uint8_t *)m.x.d[0], kq), make_rsrc((const uint8_t *)m.x.d[1], kq),
                       make_rsrc((const uint8_t *)m.x.d[2], kq)};
  const Rsrc rxs = make_rsrc((const uint8_t *)m.x.scale, 4 * live), rxm = make_rsrc((const uint8_t *)m.x.sum, 4 * live);
  const Rsrc rxq = make_rsrc((const uint8_t *)m.x.sq, m.x.normed ? 4 * live : 0);
  const RowIn rin = row_inputs(m, g, row0 + tid);  // used by threads tid < RT
  uint4 xd[3][XJ];
  uint32_t xsc[XB], xsm[XB], xsq[XB];
#pragma unroll
  for (uint32_t j = 0; j < XJ; j++) {
    const uint32_t e = (tid + j * nt) * 16;
#pragma unroll
    for (int p = 0; p < 3; p++) xd[p][j] = bl16c(rxd[p], e);
  }
#pragma unroll
  for (uint32_t j = 0; j < XB; j++) {
    const uint32_t i = 4 * (tid + j * nt);
    xsc[j] = bl4c(rxs, i);
    xsm[j] = bl4c(rxm, i);
    xsq[j] = bl4c(rxq, i);
  }
  // A CU returns load data in request order, so a wavefront that started late would find its
  // activation requests behind the other wavefronts' weight requests: a bare barrier (no
  // wait for data) puts every wavefront's activation requests ahead of all weight requests.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < DU; d++) issue(d);
  __builtin_amdgcn_sched_barrier(0);
  if (tid < MV_ZERO / 16) *(uint4 *)(lds + 16 * tid) = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (uint32_t j = 0; j < XJ; j++) {
    const uint32_t e = (tid + j * nt) * 16;
    if (e < m.ke)
#pragma unroll
      for (int p = 0; p < 3; p++) *(uint4 *)(lds + L.digits + p * m.ke + e) = xd[p][j];
  }
  // the sums of squares go to LDS by block index, so the epilogue adds them in an order that
  // does not depend on the workgroup's shape (every launch shape gives the same bits)
  float *sq = (float *)(lds + L.sq);
  const bool normed = m.x.normed != 0;
#pragma unroll
  for (uint32_t j = 0; j < XB; j++) {
    const uint32_t i = tid + j * nt;
    if (i < blocks) {
      *(float2 *)(lds + L.sm + 8 * i) = make_float2(__uint_as_float(xsc[j]) * (1.f / 64516.f), __uint_as_float(xsm[j]));
      if (normed) sq[i] = __uint_as_float(xsq[j]);
    }
  }
  for (uint32_t e = (tid + XJ * nt) * 16; e < m.ke; e += nt * 16)
#pragma unroll
    for (int p = 0; p < 3; p++) *(uint4 *)(lds + L.digits + p * m.ke + e) = bl16c(rxd[p], e);
  for (uint32_t i = tid + XB * nt; i < blocks; i += nt) {
    *(float2 *)(lds + L.sm + 8 * i) = make_float2(__uint_as_float(bl4c(rxs, 4 * i)) * (1.f / 64516.f), __uint_as_float(bl4c(rxm, 4 * i)));
    if (normed) sq[i] = __uint_as_float(bl4c(rxq, 4 * i));
  }
  __syncthreads();
  // per-lane LDS addresses of the A operands: diagonal lanes read digit p = r % 4 of their
  // group's elements, the others the zero line (the unit's reads stay below MV_ZERO); the
  // unit's offsets from the address are immediates
  const bool diag = (r >> 2) == gq && (r & 3) < 3;
  const uint32_t amask = diag ? 0xFFFFFFFFu : 0u;
  const uint32_t abase = L.digits + (r & 3) * m.ke + T::N * gq;
  const uint32_t smbase = L.sm + (T::N == 32 ? 16 * gq : 8 * gq);
  // Units are computed in chunks of DU (DU divides NSB, so a chunk never straddles a row
  // step); the per-unit code has no branches, so the compiler can overlap the LDS reads and
  // MFMAs of a chunk's units. A step's partial sums go to LDS after its last chunk.
  uint32_t cs_step = 0, cs_sl = 0;  // first unit of the next chunk
  float acc = 0.f, acc1 = 0.f;
  auto compute = [&](int slot, uint32_t sl) {
    const Unit u = unit_of(cs_step, sl);
    XA xa;
    const uint8_t *ad = lds + ((abase + T::N * u.cb) & amask);
    if (T::N == 32) {
      // columns cb + g and cb + 4 + g: 32 digits each, two 16-element blocks each
      xa.a[0][0] = *(const v4i *)(ad);
      xa.a[0][1] = *(const v4i *)(ad + 16);
      xa.a[1][0] = *(const v4i *)(ad + 128);
      xa.a[1][1] = *(const v4i *)(ad + 144);
      const float4 s0 = *(const float4 *)(lds + smbase + 8 * 2 * u.cb);
      const float4 s1 = *(const float4 *)(lds + smbase + 8 * 2 * u.cb + 64);
      xa.s[0][0] = s0.x; xa.m[0][0] = s0.y; xa.s[0][1] = s0.z; xa.m[0][1] = s0.w;
      xa.s[1][0] = s1.x; xa.m[1][0] = s1.y; xa.s[1][1] = s1.z; xa.m[1][1] = s1.w;
    } else {
      // 16-element columns cb + g and cb + 4 + g
      xa.a[0][0] = *(const v4i *)(ad);
      xa.a[1][0] = *(const v4i *)(ad + 64);
      xa.a[0][1] = xa.a[1][1] = v4i{0, 0, 0, 0};
      const float2 s0 = *(const float2 *)(lds + smbase + 8 * u.cb);
      const float2 s1 = *(const float2 *)(lds + smbase + 8 * u.cb + 32);
      xa.s[0][0] = s0.x; xa.m[0][0] = s0.y; xa.s[1][0] = s1.x; xa.m[1][0] = s1.y;
      xa.s[0][1] = xa.s[1][1] = xa.m[0][1] = xa.m[1][1] = 0.f;
    }
    acc += T::dot(buf[slot], lc, xa);
    if (GLU) acc1 += T::dot(buf1[slot], lc, xa);
  };
  auto chunk_done = [&]() {
    cs_sl += DU;
    if (cs_sl == m.NSB) {
      // step done: this lane's partial of row (rg + step * NR) * 16 + r, K slice s, group gq
      const uint32_t rr = (rg + cs_step * m.NR) * 16 + r;
      ((float *)(lds + L.vals))[(s * m.RT + rr) * 4 + gq] = acc;
      if (GLU) ((float *)(lds + L.vals1))[(s * m.RT + rr) * 4 + gq] = acc1;
      acc = 0.f; acc1 = 0.f;
      cs_sl = 0; cs_step++;
    }
  };
  // sliding window: U is a multiple of DU
  for (uint32_t u0 = DU; u0 < m.U; u0 += DU) {
#pragma unroll
    for (int d = 0; d < DU; d++) {
      compute(d, cs_sl + d);
      issue(d);
    }
    chunk_done();
  }
#pragma unroll
  for (int d = 0; d < DU; d++) compute(d, cs_sl + d);
  chunk_done();
  __syncthreads();
  if (threadIdx.x >= ((m.RT + 63) & ~63u)) return;
  float xm = 1.f;
  if (normed) {
    // lane l adds blocks 4l .. 4l + 3 (then 256 further on), and the DPP fold adds the lanes:
    // a fixed order for every launch shape (blocks is a multiple of 8)
    float tot = 0.f;
    for (uint32_t i = 4 * lane; i < blocks; i += 256) {
      const float4 q = *(const float4 *)(sq + i);
      tot += (q.x + q.y) + (q.z + q.w);
    }
    xm = 1.f / sqrtf(wave_total(tot) / (float)m.x.len + m.x.eps);
  }
  const uint32_t row = threadIdx.x;
  const bool inside = row < m.RT && row0 + row < g.rows;
  float v = 0.f, v1 = 0.f;
  if (row < m.RT) {
    for (uint32_t k = 0; k < m.NS; k++) {
      const float4 p = *(const float4 *)(lds + L.vals + 16 * (k * m.RT + row));
      v += (p.x + p.y) + (p.z + p.w);
      if (GLU) {
        const float4 p1 = *(const float4 *)(lds + L.vals1 + 16 * (k * m.RT + row));
        v1 += (p1.x + p1.y) + (p1.z + p1.w);
      }
    }
  }
  const float out = finish_row(m, g, row0 + row, inside, v * xm, v1 * xm, rin);
  if (m.arg_part) {
    // argmax key of each epilogue wavefront's rows: entry (workgroup, wavefront)
    const uint64_t k = wave_max_key(inside ? arg_key(out, row0 + row) : 0);
    if ((threadIdx.x & 63) == 0) m.arg_part[blockIdx.x * ((m.RT + 63) >> 6) + (threadIdx.x >> 6)] = k;
  }
}

// One workgroup per row tile. T1 is the chunk type of segments with kind 1 (Q and K in
// Q4_K with V in Q6_K run as one launch); both types have 32-element chunks.
template <class T0, class T1, int DU, bool GLU>
__global__ __launch_bounds__(1024) void k_mv(MV m) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // segment of this workgroup (uniform)
  uint32_t t = blockIdx.x;
  MVSeg g = m.seg[0];
  if (m.nseg > 1 && t >= m.seg[0].tiles) {
    t -= m.seg[0].tiles;
    g = m.seg[1];
    if (m.nseg > 2 && t >= m.seg[1].tiles) { t -= m.seg[1].tiles; g = m.seg[2]; }
  }
  if constexpr (std::is_same<T0, T1>::value) mv_tile<T0, DU, GLU>(m, g, t, lds);
  else if (g.kind == 0) mv_tile<T0, DU, GLU>(m, g, t, lds);
  else mv_tile<T1, DU, GLU>(m, g, t, lds);
}

// ------------------------------------------------------------------ F16 and F32 weights
//
// F16 and F32 matrices keep the GGUF row-major layout (a row is K contiguous halves or
// floats, 16-byte aligned for K % 8 == 0) and take the same QX activation, epilogues and
// launch groups as the integer kernel. A workgroup of four wavefronts owns RT rows (RT / 4
// per wavefront, four at a time): the activation is rebuilt in LDS as f32 from its digits
// (the exact integer d0 * 254^2 + d1 * 254 + d2 times scale / 254^2, as the integer kernel
// combines them), each lane reads 8 elements of each of four rows per step (one 16-byte load
// of halves, two of floats: a wavefront reads 1 or 2 KB of a row), and multiplies them in
// f32 with the activation (the reference's arithmetic, shaders.ts:39-54); the row sums are
// reduced across the wavefront and finished by the epilogue threads.
constexpr uint32_t MV16_THREADS = 256;

__device__ __forceinline__ float dot8_f16(const uint4 &w, const float4 &a, const float4 &b) {
  float s = f16lo(w.x) * a.x;
  s = fmaf(f16hi(w.x), a.y, s);
  s = fmaf(f16lo(w.y), a.z, s);
  s = fmaf(f16hi(w.y), a.w, s);
  s = fmaf(f16lo(w.z), b.x, s);
  s = fmaf(f16hi(w.z), b.y, s);
  s = fmaf(f16lo(w.w), b.z, s);
  return fmaf(f16hi(w.w), b.w, s);
}

__device__ __forceinline__ float dot8_f32(const uint4 &w0, const uint4 &w1, const float4 &a, const float4 &b) {
  float s = __uint_as_float(w0.x) * a.x;
  s = fmaf(__uint_as_float(w0.y), a.y, s);
  s = fmaf(__uint_as_float(w0.z), a.z, s);
  s = fmaf(__uint_as_float(w0.w), a.w, s);
  s = fmaf(__uint_as_float(w1.x), b.x, s);
  s = fmaf(__uint_as_float(w1.y), b.y, s);
  s = fmaf(__uint_as_float(w1.z), b.z, s);
  return fmaf(__uint_as_float(w1.w), b.w, s);
}

// ES: bytes per weight element (2: F16, 4: F32).
template <bool GLU, int ES>
__global__ __launch_bounds__(MV16_THREADS) void k_mv16(MV m) {
  extern __shared__ __attribute__((aligned(16))) float l16[];
  uint32_t t = blockIdx.x;
  MVSeg g = m.seg[0];
  if (m.nseg > 1 && t >= m.seg[0].tiles) {
    t -= m.seg[0].tiles;
    g = m.seg[1];
    if (m.nseg > 2 && t >= m.seg[1].tiles) { t -= m.seg[1].tiles; g = m.seg[2]; }
  }
  const uint32_t K = m.x.len, RT = m.RT, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float *xs = l16, *vals = xs + K, *vals1 = vals + RT, *red = vals1 + RT;
  const uint32_t row0 = t * RT;
  const RowIn rin = row_inputs(m, g, row0 + tid);  // used by threads tid < RT
  // the activation, four elements per thread and step (K % 16 == 0)
  for (uint32_t i = 4 * tid; i < K; i += 4 * MV16_THREADS) {
    const uint32_t d0 = *(const uint32_t *)(m.x.d[0] + i), d1 = *(const uint32_t *)(m.x.d[1] + i);
    const uint32_t d2 = *(const uint32_t *)(m.x.d[2] + i);
    const float sc = m.x.scale[i >> 4] * (1.f / 64516.f);
    float4 v;
    float *pv = &v.x;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int a = (int8_t)(d0 >> (8 * e)), b = (int8_t)(d1 >> (8 * e)), c = (int8_t)(d2 >> (8 * e));
      pv[e] = (float)(a * 64516 + b * 254 + c) * sc;
    }
    *(float4 *)(xs + i) = v;
  }
  if (m.x.normed) {
    float ss = 0.f;
    for (uint32_t b = tid; b < K / 16; b += MV16_THREADS) ss += m.x.sq[b];
    ss = wave_sum(ss);
    if (lane == 0) red[wv] = ss;
  }
  __syncthreads();
  const Rsrc rw = make_rsrc(g.w, g.bytes), rw1 = make_rsrc(GLU ? g.w1 : g.w, g.bytes);
  const uint32_t per = RT / 4;
  for (uint32_t r0 = wv * per; r0 < (wv + 1) * per; r0 += 4) {
    float a[4] = {0.f, 0.f, 0.f, 0.f}, a1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (uint32_t k = lane * 8; k < K; k += 512) {
      constexpr int NL = ES / 2;  // 16-byte loads per row and step
      uint4 wq[4][NL], wq1[4][NL];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        // rows past the matrix read zero (offsets past the buffer range)
        const uint32_t off = ((row0 + r0 + j) * K + k) * ES;
#pragma unroll
        for (int h = 0; h < NL; h++) {
          wq[j][h] = bl16(rw, off + 16 * h, 0);
          if (GLU) wq1[j][h] = bl16(rw1, off + 16 * h, 0);
        }
      }
      const float4 x0 = *(const float4 *)(xs + k), x1 = *(const float4 *)(xs + k + 4);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (ES == 2) {
          a[j] += dot8_f16(wq[j][0], x0, x1);
          if (GLU) a1[j] += dot8_f16(wq1[j][0], x0, x1);
        } else {
          a[j] += dot8_f32(wq[j][0], wq[j][NL - 1], x0, x1);
          if (GLU) a1[j] += dot8_f32(wq1[j][0], wq1[j][NL - 1], x0, x1);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float v = wave_sum(a[j]);
      const float v1 = GLU ? wave_sum(a1[j]) : 0.f;
      if (lane == 0) {
        vals[r0 + j] = v;
        if (GLU) vals1[r0 + j] = v1;
      }
    }
  }
  __syncthreads();
  if (tid >= ((RT + 63) & ~63u)) return;
  float xm = 1.f;
  if (m.x.normed) xm = 1.f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + m.x.eps);
  const bool inside = tid < RT && row0 + tid < g.rows;
  const float v = tid < RT ? vals[tid] : 0.f, v1 = (GLU && tid < RT) ? vals1[tid] : 0.f;
  const float out = finish_row(m, g, row0 + tid, inside, v * xm, v1 * xm, rin);
  if (m.arg_part) {
    const uint64_t k = wave_max_key(inside ? arg_key(out, row0 + tid) : 0);
    if ((tid & 63) == 0) m.arg_part[blockIdx.x * ((RT + 63) >> 6) + (tid >> 6)] = k;
  }
}

// ------------------------------------------------------------------ host side

uint64_t qx_bytes(uint32_t K) {
  const uint64_t kp = (K + 63) / 64 * 64;
  return 3 * kp + 12 * (kp / 16);
}

QXOut qx_view(void *base, uint32_t K) {
  const uint64_t kp = (K + 63) / 64 * 64;
  uint8_t *p = (uint8_t *)base;
  QXOut q;
  q.d0 = (int8_t *)p; q.d1 = (int8_t *)(p + kp); q.d2 = (int8_t *)(p + 2 * kp);
  q.scale = (float *)(p + 3 * kp);
  q.sum = q.scale + kp / 16;
  q.sq = q.sum + kp / 16;
  return q;
}

QXView qx_const(const QXOut &q, uint32_t K, bool normed, float eps) {
  QXView v;
  v.d[0] = q.d0; v.d[1] = q.d1; v.d[2] = q.d2;
  v.scale = q.scale; v.sum = q.sum; v.sq = q.sq;
  v.normed = normed ? 1u : 0u; v.len = K; v.eps = eps;
  return v;
}

hipError_t quantize(hipStream_t s, const float *x, uint32_t K, const float *norm_w, const QXOut &q) {
  if (!K || K % 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_quantize, dim3((K + 255) / 256), dim3(256), 0, s, x, K, norm_w, q);
  return hipGetLastError();
}

static bool float_type(int t) { return t == F16 || t == F32; }
static uint32_t float_bytes(int t) { return t == F32 ? 4 : 2; }

// F16 / F32 rows of up to 32768 elements (the f32 activation fits in LDS), 32-bit buffer
// offsets.
static bool mv16_supported(const Matrix &w) {
  return float_type(w.type) && w.layout == LAYOUT_GGUF && w.cols && w.rows && w.cols % 16 == 0 && w.cols <= 32768 &&
         ((uint64_t)w.rows + 64) * w.cols * float_bytes(w.type) < (1ull << 31);
}

// Row tiles of 64, 32 or 16 rows: the largest that still gives every CU a workgroup.
static MVPlan mv16_plan(const Matrix &w, const uint32_t *rows, uint32_t n) {
  const uint32_t cus = (uint32_t)device_cu_count();
  MVPlan p{};
  for (uint32_t rt = 64; rt >= 16; rt /= 2) {
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < n; i++) tiles += (rows[i] + rt - 1) / rt;
    p.RT = rt;
    p.tiles = tiles;
    if (tiles >= cus) break;
  }
  p.C = w.cols; p.NS = p.NSB = p.NR = p.ITER = p.DU = 1;
  p.threads = MV16_THREADS;
  p.lds = 4 * (w.cols + 2 * p.RT + 4);
  return p;
}

bool mv_supported(const Matrix &w) {
  if (float_type(w.type)) return mv16_supported(w);
  if (w.layout != LAYOUT_PLANAR || !w.cols || !w.rows) return false;
  if (w.type == Q4_K || w.type == Q5_K || w.type == Q6_K) return w.cols % 256 == 0;
  if (w.type == Q8_0 || w.type == Q4_0) return w.cols % 32 == 0;
  return false;
}

bool mv_mixable(int a, int b) {
  if (a == b) return true;
  if (a > b) std::swap(a, b);
  return (a == Q4_K || a == Q5_K) && b == Q6_K;
}

static uint32_t lds_limit() { return LDS_MAX; }

uint32_t mv_arg_entries(const Matrix &w) {
  const MVPlan p = mv_plan(w, &w.rows, 1, false, false, true);
  return p.tiles * ((p.RT + 63) / 64);
}

// The launch shape, searched over the K split (NS slices of NSB 8-column units), the row
// tiles (NR groups of ITER steps) and the pipeline depth DU (a divisor of the units per
// wavefront). The cost is the rows the busiest CU streams (whole rounds of CU-count tiles),
// stretched when a CU holds less than ~64 KB of weight loads in flight (more than ~100 KB
// only queues), when the activation staging is amortised over few rows, and for idle chunk
// columns.
MVPlan mv_plan(const Matrix &w, const uint32_t *rows, uint32_t n, bool glu, bool quantized_out, bool normed) {
  if (float_type(w.type)) return mv16_plan(w, rows, n);
  MVPlan best_p{};
  const uint32_t N = chunk_elems(w.type), C = w.cols / N, CQ = (C + 7) / 8;
  const uint32_t cus = (uint32_t)device_cu_count();
  const uint32_t dumax = glu ? 2 : 4;
  // unique weight bytes of one unit (16 rows x 8 chunk columns and its scale planes), KB
  const double unit_kb = w.type == Q6_K ? 2.625 : w.type == Q5_K ? 2.75 : w.type == Q8_0 ? 2.125 : 2.25;
  double best_cost = 1e30;
  for (uint32_t ns = 1; ns <= 16; ns++) {
    const uint32_t nsb = (CQ + ns - 1) / ns;
    if ((nsb - 1) * ns >= CQ && ns > 1) continue;  // a slice would be empty
    const uint32_t waste = ns * nsb * 8 - C;
    if (waste * 7 > C && ns > 1) continue;
    const uint32_t ke = ns * nsb * 8 * N;
    for (uint32_t nr = 1; nr * ns <= 16; nr++) {
      for (uint32_t iter = 1; iter <= 256; iter++) {
        const uint32_t rt = 16 * nr * iter;
        if (rt > 64 * nr * ns || rt > 1024) break;  // one epilogue thread per row
        if (quantized_out && rt % 16) continue;
        const LdsMap lm = lds_map(ke, ns, rt, glu, normed);
        if (lm.bytes > lds_limit()) break;
        const uint32_t units = iter * nsb;
        uint32_t tiles = 0;
        for (uint32_t i = 0; i < n; i++) tiles += (rows[i] + rt - 1) / rt;
        const uint32_t rounds = (tiles + cus - 1) / cus;
        const uint32_t per_cu = lm.bytes > 80 * 1024 ? 1 : 2;
        const double resident = tiles >= per_cu * cus ? (double)per_cu : tiles > cus ? (double)tiles / cus : 1.0;
        auto inflight = [&](uint32_t du) {
          return (double)(nr * ns) * (units < du ? units : du) * (glu ? 2 : 1) * unit_kb * resident;
        };
        // deepest pipeline (a divisor of NSB, so a window of DU units stays in one row step)
        // that keeps a CU's loads in flight within ~100 KB
        uint32_t du = dumax;
        while (du > 1 && (nsb % du || inflight(du) > 100.0)) du /= 2;
        double cost = (double)rounds * rt * (1.0 + (double)waste / C);
        if (inflight(du) < 64.0) cost *= 64.0 / inflight(du);
        cost *= 1.0 + 2.0 / rt;  // activation staging per workgroup
        if (cost < best_cost) {
          best_cost = cost;
          MVPlan p{};
          p.C = C; p.NS = ns; p.NSB = nsb; p.NR = nr; p.ITER = iter; p.DU = du; p.RT = rt; p.tiles = tiles;
          p.threads = 64 * nr * ns; p.lds = lm.bytes;
          best_p = p;
        }
        if (tiles <= cus) break;  // more steps only lengthen the tile
      }
    }
  }
  return best_p;
}

template <class T0, class T1, bool GLU>
static hipError_t launch_t(hipStream_t s, const MV &m, const MVPlan &p) {
  const dim3 grid(p.tiles), block(p.threads);
  auto go = [&](auto kernel) -> hipError_t {
    if (p.lds > 64 * 1024) lds_opt_in((const void *)kernel);
    hipLaunchKernelGGL(kernel, grid, block, p.lds, s, m);
    return hipGetLastError();
  };
  switch (p.DU) {
    case 1: return go(k_mv<T0, T1, 1, GLU>);
    case 2: return go(k_mv<T0, T1, 2, GLU>);
    case 4: if constexpr (!GLU) return go(k_mv<T0, T1, 4, GLU>); else break;
  }
  return hipErrorInvalidValue;
}

// Launch shapes measured by mv_tune, per device and launch signature (weight types, K, the
// segments' rows, gated pair, epilogue, re-quantized output).
namespace {
typedef std::tuple<int, int, int, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, bool, int, bool> PlanKey;
std::mutex g_plan_mu;
std::map<PlanKey, MVPlan> g_plans;

PlanKey plan_key(const MVTarget *t, uint32_t n, int epi, bool qout) {
  int t1 = t[0].w->type;
  for (uint32_t i = 0; i < n; i++)
    if (t[i].w->type != t[0].w->type) t1 = t[i].w->type;
  int dev = 0;
  hipGetDevice(&dev);
  return PlanKey(dev, t[0].w->type, t1, t[0].w->cols, n, t[0].w->rows, n > 1 ? t[1].w->rows : 0, n > 2 ? t[2].w->rows : 0,
                 t[0].w1 != nullptr, epi, qout);
}
}  // namespace

static hipError_t mv_launch(hipStream_t s, const MVTarget *t, uint32_t n, const QXView &x, int epi, const MVOut *out,
                            const MVPlan *forced);

hipError_t mv(hipStream_t s, const MVTarget *t, uint32_t n, const QXView &x, int epi, const MVOut *out) {
  return mv_launch(s, t, n, x, epi, out, nullptr);
}

// Holds the stream for `ticks` of the constant-rate wall clock, so the launches queued
// behind it run back to back however slowly the host submits them (a profiler, a busy host).
// Bounded: the loop also ends after 2^16 sleeps.
__global__ void k_hold(long long ticks) {
  const long long t0 = wall_clock64();
  for (uint32_t i = 0; i < (1u << 16) && wall_clock64() - t0 < ticks; i++) __builtin_amdgcn_s_sleep(63);
}

// Candidates keep the cost model's K split (NS slices of NSB units, so the staged activation
// and the order in which every row's products are summed do not change: all candidates give
// the same bits) and vary the rows per workgroup (NR groups of ITER steps) and the pipeline
// depth DU. Each is timed with HIP events over back-to-back launches that rotate through the
// sets (so the weights come from HBM, not a cache); the fastest is kept for the signature.
// The launch shapes mv_tune times for one signature: the cost model's plan first, then every
// other (NR, ITER, DU) with the model's K split.
static std::vector<MVPlan> mv_candidates(const MVTarget *t, uint32_t n, const QXView &x, bool qout) {
  const Matrix &w0 = *t[0].w;
  const bool glu = t[0].w1 != nullptr;
  uint32_t rows[MV_MAX_SEGS];
  for (uint32_t i = 0; i < n; i++) rows[i] = t[i].w->rows;
  const MVPlan base = mv_plan(w0, rows, n, glu, qout, x.normed != 0);
  if (!base.RT) return {};
  const uint32_t ke = base.NS * base.NSB * 8 * chunk_elems(w0.type);
  std::vector<MVPlan> cands{base};
  for (uint32_t nr = 1; nr * base.NS <= 16; nr++)
    for (uint32_t it = 1; it <= 8; it++) {
      const uint32_t rt = 16 * nr * it;
      if (rt > 64 * nr * base.NS || rt > 1024) break;
      const uint32_t lds = lds_map(ke, base.NS, rt, glu, x.normed != 0).bytes;
      if (lds > lds_limit()) break;
      uint32_t tiles = 0;
      for (uint32_t i = 0; i < n; i++) tiles += (rows[i] + rt - 1) / rt;
      if (tiles > 4096) continue;
      for (uint32_t du : {1u, 2u, 4u}) {
        if (base.NSB % du || (glu && du > 2)) continue;
        MVPlan p = base;
        p.NR = nr; p.ITER = it; p.DU = du; p.RT = rt; p.tiles = tiles; p.threads = 64 * nr * base.NS; p.lds = lds;
        if (p.NR != base.NR || p.ITER != base.ITER || p.DU != base.DU) cands.push_back(p);
      }
    }
  return cands;
}

hipError_t mv_shapes(hipStream_t s, const Matrix &w, const QXView &x, float *y, uint32_t max_shapes, uint32_t *count) {
  MVTarget t; t.w = &w; t.w1 = nullptr; t.y = y;
  const std::vector<MVPlan> cands = float_type(w.type) ? std::vector<MVPlan>{} : mv_candidates(&t, 1, x, false);
  *count = (uint32_t)std::min<size_t>(cands.size(), max_shapes);
  for (uint32_t k = 0; k < *count; k++) {
    t.y = y + (uint64_t)k * w.rows;
    const hipError_t e = mv_launch(s, &t, 1, x, MV_STORE, nullptr, &cands[k]);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t mv_tune(hipStream_t s, const MVTarget *sets, uint32_t nsets, uint32_t n, const QXView &x, int epi,
                   const MVOut *out) {
  if (!nsets || n < 1 || n > (uint32_t)MV_MAX_SEGS) return hipErrorInvalidValue;
  const Matrix &w0 = *sets[0].w;
  if (float_type(w0.type) || (out && out->arg_part)) return hipSuccess;  // F16/F32 and the head keep the model's plan
  const bool qout = out && out->q.d0;
  const PlanKey key = plan_key(sets, n, epi, qout);
  {
    std::lock_guard<std::mutex> lock(g_plan_mu);
    if (g_plans.count(key)) return hipSuccess;
  }
  const std::vector<MVPlan> cands = mv_candidates(sets, n, x, qout);
  if (cands.empty()) return hipErrorInvalidValue;
  const MVPlan &base = cands[0];
  hipEvent_t e0 = nullptr, e1 = nullptr;
  WGD_HIP(hipEventCreate(&e0));
  hipError_t err = hipEventCreate(&e1);
  int dev = 0, khz = 0;
  if (err == hipSuccess) err = hipGetDevice(&dev);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
  MVPlan best = base;
  double best_us = 1e30;
  const uint32_t reps = nsets < 8 ? 16 : 2 * nsets;
  double hold_us = 50.0 + 8.0 * reps;  // longer than the host takes to queue the timed launches
  for (const MVPlan &p : cands) {
    float ms = 0.f;
    for (int attempt = 0; attempt < 4 && err == hipSuccess; attempt++) {
      for (uint32_t i = 0; i < 2 && err == hipSuccess; i++) err = mv_launch(s, sets + n * (i % nsets), n, x, epi, out, &p);
      if (err == hipSuccess) {
        hipLaunchKernelGGL(k_hold, dim3(1), dim3(64), 0, s, (long long)(hold_us * khz / 1000.0));
        err = hipGetLastError();
      }
      const auto t0 = std::chrono::steady_clock::now();
      if (err == hipSuccess) err = hipEventRecord(e0, s);
      for (uint32_t i = 0; i < reps && err == hipSuccess; i++) err = mv_launch(s, sets + n * (i % nsets), n, x, epi, out, &p);
      if (err == hipSuccess) err = hipEventRecord(e1, s);
      const double queued_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
      if (err == hipSuccess) err = hipEventSynchronize(e1);
      if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
      if (queued_us < 0.7 * hold_us) break;  // every timed launch was queued before the hold ended
      hold_us = std::min(2.0 * queued_us + 50.0, 200000.0);
    }
    // a candidate must beat the cost model's plan by more than timing noise
    const double us = (double)ms * 1e3 / reps * (&p == &cands[0] ? 0.98 : 1.0);
    if (err == hipSuccess && us < best_us) { best_us = us; best = p; }
  }
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  if (err != hipSuccess) return err;
  std::lock_guard<std::mutex> lock(g_plan_mu);
  g_plans[key] = best;
  return hipSuccess;
}

static hipError_t mv_launch(hipStream_t s, const MVTarget *t, uint32_t n, const QXView &x, int epi, const MVOut *out,
                            const MVPlan *forced) {
  if (n < 1 || n > (uint32_t)MV_MAX_SEGS) return hipErrorInvalidValue;
  const Matrix &w0 = *t[0].w;
  const bool glu = t[0].w1 != nullptr;
  const bool qout = out && out->q.d0;
  if (qout && n != 1) return hipErrorInvalidValue;
  if ((epi == MV_SILU || epi == MV_GELU) != glu) return hipErrorInvalidValue;
  if (x.len != w0.cols) return hipErrorInvalidValue;
  uint32_t rows[MV_MAX_SEGS];
  if (float_type(w0.type)) {
    for (uint32_t i = 0; i < n; i++) {
      const Matrix &w = *t[i].w;
      if (!mv16_supported(w) || w.type != w0.type || w.cols != w0.cols || !t[i].y || (t[i].w1 != nullptr) != glu)
        return hipErrorInvalidValue;
      if (glu && (t[i].w1->type != w.type || t[i].w1->layout != w.layout || t[i].w1->cols != w.cols ||
                  t[i].w1->rows != w.rows))
        return hipErrorInvalidValue;
      rows[i] = w.rows;
    }
    const MVPlan p = mv16_plan(w0, rows, n);
    if (p.lds > lds_limit()) return hipErrorInvalidValue;
    MV m{};
    m.nseg = n;
    for (uint32_t i = 0; i < n; i++) {
      MVSeg &g = m.seg[i];
      g.w = t[i].w->data; g.w1 = glu ? t[i].w1->data : nullptr;
      g.bytes = (uint32_t)((uint64_t)rows[i] * w0.cols * float_bytes(w0.type));
      g.y = t[i].y; g.bias = t[i].bias; g.rows = rows[i];
      g.tiles = (rows[i] + p.RT - 1) / p.RT;
    }
    m.x = x; m.C = w0.cols; m.ke = w0.cols; m.RT = p.RT; m.NS = m.NSB = m.NR = m.ITER = m.U = 1;
    m.epi = epi;
    if (qout) { m.oq = out->q; m.oq_norm = out->norm_w; }
    if (out && out->arg_part) {
      if (n != 1) return hipErrorInvalidValue;
      m.arg_part = out->arg_part;
    }
    auto go = [&](auto kernel) -> hipError_t {
      if (p.lds > 64 * 1024) lds_opt_in((const void *)kernel);
      hipLaunchKernelGGL(kernel, dim3(p.tiles), dim3(MV16_THREADS), p.lds, s, m);
      return hipGetLastError();
    };
    if (w0.type == F32) return glu ? go(k_mv16<true, 4>) : go(k_mv16<false, 4>);
    return glu ? go(k_mv16<true, 2>) : go(k_mv16<false, 2>);
  }
  // Q6_K segments may share a launch with Q4_K or Q5_K ones (same chunk shape); other
  // types run alone
  int other = -1;
  for (uint32_t i = 0; i < n; i++) {
    const Matrix &w = *t[i].w;
    if (w.type != w0.type) {
      if ((other >= 0 && w.type != other) || !mv_mixable(w0.type, w.type) || glu) return hipErrorInvalidValue;
      other = w.type;
    }
    if (!mv_supported(w) || w.cols != w0.cols || !t[i].y) return hipErrorInvalidValue;
    if ((t[i].w1 != nullptr) != glu) return hipErrorInvalidValue;
    if (glu) {
      const Matrix &w1 = *t[i].w1;
      if (w1.type != w.type || w1.layout != w.layout || w1.cols != w.cols || w1.rows != w.rows) return hipErrorInvalidValue;
    }
    rows[i] = w.rows;
  }
  MVPlan p{};
  if (forced) {
    p = *forced;
  } else {
    std::lock_guard<std::mutex> lock(g_plan_mu);
    const auto it = g_plans.find(plan_key(t, n, epi, qout));
    if (it != g_plans.end()) p = it->second;
  }
  if (!p.RT) p = mv_plan(w0, rows, n, glu, qout, x.normed != 0);
  if (!p.RT || p.threads != 64 * p.NS * p.NR || p.threads > 1024 || p.RT > p.threads || p.NSB % p.DU ||
      p.lds > lds_limit() || (qout && p.RT % 16))
    return hipErrorInvalidValue;
  MV m{};
  m.nseg = n;
  for (uint32_t i = 0; i < n; i++) {
    const Matrix &w = *t[i].w;
    MVSeg &g = m.seg[i];
    g.w = w.data; g.w1 = glu ? t[i].w1->data : nullptr;
    g.bpr = w.cols / block_size(w.type);
    const uint64_t nbp = (uint64_t)g.bpr * tile_rows(w.rows), bytes = planar_bytes(w.type, w.cols, w.rows);
    if (bytes >= (1ull << 31)) return hipErrorInvalidValue;  // 32-bit buffer offsets with headroom
    g.nbp = (uint32_t)nbp;
    g.bytes = (uint32_t)bytes;
    g.y = t[i].y; g.bias = t[i].bias;
    g.kind = w.type == w0.type ? 0u : 1u;
    g.rows = w.rows;
    g.tiles = (w.rows + p.RT - 1) / p.RT;
  }
  m.x = x;
  m.C = p.C;
  m.ke = p.NS * p.NSB * 8 * chunk_elems(w0.type);
  m.NS = p.NS; m.NSB = p.NSB; m.NR = p.NR; m.ITER = p.ITER; m.RT = p.RT; m.U = p.ITER * p.NSB;
  m.epi = epi;
  m.oq = QXOut{};
  m.oq_norm = nullptr;
  m.arg_part = nullptr;
  if (qout) { m.oq = out->q; m.oq_norm = out->norm_w; }
  if (out && out->arg_part) {
    if (n != 1) return hipErrorInvalidValue;
    m.arg_part = out->arg_part;
  }
  if (other >= 0) {
    if (w0.type == Q4_K) return launch_t<CQ4K, CQ6K, false>(s, m, p);
    if (w0.type == Q5_K) return launch_t<CQ5K, CQ6K, false>(s, m, p);
    if (other == Q4_K) return launch_t<CQ6K, CQ4K, false>(s, m, p);
    return launch_t<CQ6K, CQ5K, false>(s, m, p);
  }
  switch (w0.type) {
    case Q4_K: return glu ? launch_t<CQ4K, CQ4K, true>(s, m, p) : launch_t<CQ4K, CQ4K, false>(s, m, p);
    case Q5_K: return glu ? launch_t<CQ5K, CQ5K, true>(s, m, p) : launch_t<CQ5K, CQ5K, false>(s, m, p);
    case Q6_K: return glu ? launch_t<CQ6K, CQ6K, true>(s, m, p) : launch_t<CQ6K, CQ6K, false>(s, m, p);
    case Q8_0: return glu ? launch_t<CQ80, CQ80, true>(s, m, p) : launch_t<CQ80, CQ80, false>(s, m, p);
    case Q4_0: return glu ? launch_t<CQ40, CQ40, true>(s, m, p) : launch_t<CQ40, CQ40, false>(s, m, p);
  }
  return hipErrorInvalidValue;
}

}  // namespace wgd
