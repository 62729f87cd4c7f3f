// matvec.hip — decode dequant-matvec (batch 1) for gfx950 on integer dot products.
//
// Replaces matmulShader (src/core/shaders.ts:39-54) for one activation row. The reference
// decodes every weight to f32 and multiplies by an f32 activation. Here the activation row
// is quantized first ("QX" format): per 16-element block a scale s = max|x| / 127 and three
// signed base-254 digits per element, x = s * (d0 + d1/254 + d2/254^2) (error <= 6.1e-8 *
// max|x|, f32-level). Weights are consumed in their raw form: 4-bit (Q4_K), 6-bit (Q6_K) or
// 8-bit (Q8_0) quants are masked into bytes and multiplied with the digits by
// v_dot4_i32_i8, four products per instruction, exact in int32. Block scales apply once per
// 16 elements; the Q4_K minimum and the Q6_K offset use the exact sums of x.
//
// Memory: the weights are stored in "chunks" (planar layouts, quant.hip): the quants of 32
// consecutive elements of a row (16 for Q8_0) in 16 bytes, a row's chunks consecutive, the
// per-block headers in separate planes. A lane owns a chunk column and every load
// instruction of a wavefront reads Wc consecutive chunks of P = 64/Wc rows: 1 KB of
// contiguous bytes for Wc = 64. Each wavefront keeps D row steps of loads in flight
// (software pipeline over registers) and the activation digits of its chunk columns in
// registers for all of its rows.
//
// Work split: a workgroup owns RT rows; NS wavefronts split K, NR wavefronts split the rows.
// Per row step the lanes of a row are summed with DPP adds, the K slices through LDS
// in slice order (deterministic), and the first RT threads run the epilogue: store, residual
// add, or the gated SwiGLU/GeGLU of a gate/up pair, optionally re-quantizing the result
// (times the next RMSNorm weight) for the next matvec. Nothing synchronizes across
// workgroups inside a launch: on MI355X each XCD has its own L2, and device-scope fences
// write back and invalidate it.
#include <cstdlib>

#include "internal.h"
#include "decode.h"
#include "matvec.h"

namespace wgd {

// ------------------------------------------------------------------ quantization helpers

// Quantizes one value per lane in aligned 16-lane groups; the block scale is max|v| / 127.
__device__ __forceinline__ void quant_lane16(float v, float &scale, int &d0, int &d1, int &d2) {
  float a = fabsf(v);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
  scale = a * (1.f / 127.f);
  const float u = a > 0.f ? v * (127.f / a) : 0.f;
  const float r0 = fminf(fmaxf(rintf(u), -127.f), 127.f);
  const float t = (u - r0) * 254.f;
  const float r1 = fminf(fmaxf(rintf(t), -127.f), 127.f);
  const float t2 = (t - r1) * 254.f;
  const float r2 = fminf(fmaxf(rintf(t2), -127.f), 127.f);
  d0 = (int)r0; d1 = (int)r1; d2 = (int)r2;
}

// Writes element `i` of a QX vector: v is the stored value (already times any norm
// weight), raw the value whose square is summed. Lanes hold 16 consecutive aligned elements.
__device__ __forceinline__ void qx_store(const QXOut &q, uint32_t i, float v, float raw, bool live) {
  float sc; int d0, d1, d2;
  quant_lane16(live ? v : 0.f, sc, d0, d1, d2);
  float s16 = live ? v : 0.f, q16 = live ? raw * raw : 0.f;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) { s16 += __shfl_xor(s16, o, 64); q16 += __shfl_xor(q16, o, 64); }
  if (live) {
    q.d0[i] = (int8_t)d0; q.d1[i] = (int8_t)d1; q.d2[i] = (int8_t)d2;
    if ((i & 15) == 0) { q.scale[i >> 4] = sc; q.sum[i >> 4] = s16; q.sq[i >> 4] = q16; }
  }
}

// Standalone quantization of x (length K), optionally as x * w: one workgroup per 256.
__global__ __launch_bounds__(256) void k_quantize(const float *x, uint32_t K, const float *w, QXOut q) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  const bool live = i < K;
  const float v = live ? x[i] : 0.f;
  qx_store(q, i, (live && w) ? v * w[i] : v, v, live);
}

// ------------------------------------------------------------------ chunk kernels

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Activation digits used by the matvec. Two (x within 1.6e-5 * max|x| of its block) exceed
// a 1e-3 relative logits bound at the 8B decoder shape; three are f32-level.
constexpr int DIG = 3;

// Weight loads: raw buffer loads over the matrix allocation (a 128-bit resource in SGPRs),
// with the per-lane chunk offset in a VGPR and the per-row-step offset in an SGPR, so the
// address arithmetic is scalar; offsets past the allocation read zero. Non-temporal (nt):
// weight bytes are read once per token.
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
__device__ __forceinline__ uint32_t bl2(Rsrc r, uint32_t v, uint32_t s) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, v, s, CPOL_NT);
}
__device__ __forceinline__ float f16lo(uint32_t v) { return __half2float(__ushort_as_half((unsigned short)(v & 0xFFFFu))); }

// Activation of one chunk column: N = 32 (two 16-element blocks) or 16 elements.
template <int N> struct XS {
  int d[DIG][N / 4];
  float s[N / 16], m[N / 16];  // block scales, block sums
  float ss;                    // sum of squares (normed vectors)
};
template <int N>
__device__ __forceinline__ void load_xs(const QXView &x, uint32_t c, XS<N> &o) {
#pragma unroll
  for (int p = 0; p < DIG; p++)
#pragma unroll
    for (int h = 0; h < N / 16; h++) {
      const int4 v = *(const int4 *)(x.d[p] + N * c + 16 * h);
      o.d[p][4 * h] = v.x; o.d[p][4 * h + 1] = v.y; o.d[p][4 * h + 2] = v.z; o.d[p][4 * h + 3] = v.w;
    }
  o.ss = 0.f;
#pragma unroll
  for (int h = 0; h < N / 16; h++) {
    o.s[h] = x.scale[(N / 16) * c + h] * (1.f / 64516.f);  // digit sums come weighted by 254^2
    o.m[h] = x.sum[(N / 16) * c + h];
    if (x.normed) o.ss += x.sq[(N / 16) * c + h];
  }
}

// Q4_K chunk: sub-block j of a block; byte i = q[i] | q[i + 16] << 4. Header plane: the
// GGUF header (d, dmin, 12 bytes of packed 6-bit scales/mins, quant.ts:10-16).
// Chunk ci = step + lane (step = first row of the step x C, a multiple of 8).
struct CQ4K {
  static constexpr int N = 32;
  struct W { uint4 q, h; };
  // Lane constants: load offsets and the scale/min unpack of sub-block j = c % 8.
  struct L { uint32_t vq, vh; bool lo; uint32_t sa, wa, sb, wb, sc, wc; };
  static __device__ __forceinline__ L lane(uint32_t c, uint32_t lane_ci) {
    const uint32_t j = c & 7;
    L l;
    l.vq = 16 * lane_ci;
    l.vh = 16 * (lane_ci >> 3);
    l.lo = j < 4;
    if (j < 4) { l.sa = 8 * j; l.wa = 6; l.sb = 0; l.wb = 0; l.sc = 8 * j; l.wc = 6; }
    else { l.sa = 8 * (j - 4); l.wa = 4; l.sb = 8 * (j - 4) + 6; l.wb = 2; l.sc = 8 * (j - 4) + 4; l.wc = 4; }
    return l;
  }
  static __device__ __forceinline__ W load(Rsrc r, uint32_t nbt, uint32_t step, const L &l) {
    W w;
    w.q = bl16(r, l.vq, 16 * step);
    w.h = bl16(r, l.vh, nbt * 128 + 2 * step);
    return w;
  }
  // Digit sums of 16 elements of 4-bit weights fit int32 when weighted by 254^2, 254, 1
  // (|d0 sum| <= 16 * 15 * 127): one integer combine per half, one conversion.
  static __device__ __forceinline__ int icombine(const int *sd) {
    return __mul24(sd[0], 64516) + __mul24(sd[1], 254) + sd[2];
  }
  static __device__ __forceinline__ float dot(const W &r, const L &l, const XS<32> &x) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    int lo[DIG] = {}, hi[DIG] = {};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int a = (int)(q[k] & 0x0F0F0F0Fu), b = (int)((q[k] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int p = 0; p < DIG; p++) { lo[p] = dot4(a, x.d[p][k], lo[p]); hi[p] = dot4(b, x.d[p][4 + k], hi[p]); }
    }
    // scale/min of sub-block j (quant.ts:15-16)
    const uint32_t A = l.lo ? r.h.y : r.h.w, B = l.lo ? r.h.z : r.h.w;
    const uint32_t sc = __builtin_amdgcn_ubfe(A, l.sa, l.wa) | (__builtin_amdgcn_ubfe(r.h.y, l.sb, l.wb) << 4);
    const uint32_t mn = __builtin_amdgcn_ubfe(B, l.sc, l.wc) | (__builtin_amdgcn_ubfe(r.h.z, l.sb, l.wb) << 4);
    const float d = f16lo(r.h.x), dm = f16lo(r.h.x >> 16);
    // x.s holds the block scales divided by 254^2
    const float S = x.s[0] * (float)icombine(lo) + x.s[1] * (float)icombine(hi);
    return d * (float)sc * S - dm * (float)mn * (x.m[0] + x.m[1]);
  }
};

// Q6_K chunk: ql byte i = lo4[i] | lo4[i + 16] << 4; qh dword m byte b holds the high 2 bits
// of elements 8m+b, 16+8m+b, 8m+4+b, 16+8m+4+b at bits 0, 2, 4, 6; two int8 scales (one per
// 16 elements) and the block's f16 d in their planes (quant.ts:21-27).
struct CQ6K {
  static constexpr int N = 32;
  struct W { uint4 q; uint2 h; uint32_t s, d; };
  struct L { uint32_t vq, vh, vs, vd; };
  static __device__ __forceinline__ L lane(uint32_t, uint32_t lane_ci) {
    return L{16 * lane_ci, 8 * lane_ci, 2 * lane_ci, 2 * (lane_ci >> 3)};
  }
  static __device__ __forceinline__ W load(Rsrc r, uint32_t nbt, uint32_t step, const L &l) {
    W w;
    w.q = bl16(r, l.vq, 16 * step);
    w.h = bl8(r, l.vh, nbt * 128 + 8 * step);
    w.s = bl2(r, l.vs, nbt * 192 + 2 * step);
    w.d = bl2(r, l.vd, nbt * 208 + step / 4);
    return w;
  }
  static __device__ __forceinline__ float dot(const W &r, const L &, const XS<32> &x) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    int lo[DIG] = {}, hi[DIG] = {};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t Q = (k < 2 ? r.h.x : r.h.y) >> (4 * (k & 1));
      const int a = (int)((q[k] & 0x0F0F0F0Fu) | ((Q << 4) & 0x30303030u));
      const int b = (int)(((q[k] >> 4) & 0x0F0F0F0Fu) | ((Q << 2) & 0x30303030u));
#pragma unroll
      for (int p = 0; p < DIG; p++) { lo[p] = dot4(a, x.d[p][k], lo[p]); hi[p] = dot4(b, x.d[p][4 + k], hi[p]); }
    }
    const float s0 = (float)(int8_t)(r.s & 0xFFu), s1 = (float)(int8_t)((r.s >> 8) & 0xFFu);
    // 6-bit sums overflow the 254^2 weighting: combine the first two digits in integers
    const float cl = (float)(__mul24(lo[0], 254) + lo[1]) * 254.f + (float)lo[2];
    const float ch = (float)(__mul24(hi[0], 254) + hi[1]) * 254.f + (float)hi[2];
    const float S = s0 * (x.s[0] * cl - 32.f * x.m[0]) + s1 * (x.s[1] * ch - 32.f * x.m[1]);
    return f16lo(r.d) * S;
  }
};

// Q8_0 chunk: half a block, 16 int8 quants; the block's f16 d in its plane (quant.ts:8).
struct CQ80 {
  static constexpr int N = 16;
  struct W { uint4 q; uint32_t d; };
  struct L { uint32_t vq, vd; };
  static __device__ __forceinline__ L lane(uint32_t, uint32_t lane_ci) { return L{16 * lane_ci, 2 * (lane_ci >> 1)}; }
  static __device__ __forceinline__ W load(Rsrc r, uint32_t nbt, uint32_t step, const L &l) {
    W w;
    w.q = bl16(r, l.vq, 16 * step);
    w.d = bl2(r, l.vd, nbt * 32 + step);
    return w;
  }
  static __device__ __forceinline__ float dot(const W &r, const L &, const XS<16> &x) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    int s[DIG] = {};
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int p = 0; p < DIG; p++) s[p] = dot4((int)q[k], x.d[p][k], s[p]);
    const float c = (float)(__mul24(s[0], 254) + s[1]) * 254.f + (float)s[2];
    return f16lo(r.d) * x.s[0] * c;
  }
};

// ------------------------------------------------------------------ the tile kernel

__device__ __forceinline__ float gelu_tanh_mv(float g) {
  return 0.5f * g * (1.f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g)));
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

// Epilogue of one row: thread t < RT holds row row0 + t of segment g.
__device__ __forceinline__ void finish_row(const MV &m, const MVSeg &g, uint32_t row, bool live, float v, float u) {
  float out = 0.f;
  if (live) {
    if (g.bias) v += g.bias[row];
    float *dst = g.y + row;
    switch (m.epi) {
      case MV_STORE: out = v; break;
      case MV_ADD: out = *dst + v; break;
      case MV_SILU: out = v / (1.f + expf(-v)) * u; break;
      case MV_GELU: out = gelu_tanh_mv(v) * u; break;
    }
    *dst = out;
  }
  if (m.oq.d0) {
    const float wn = (live && m.oq_norm) ? m.oq_norm[row] : 1.f;
    qx_store(m.oq, row, out * wn, out, live);
  }
}

// Wavefronts per workgroup: up to 16 when a lane owns one chunk column and keeps at most 8
// chunk loads in flight (four waves per SIMD, 128 VGPRs), else 8 (two per SIMD, 256 VGPRs).
constexpr uint32_t MV_MAX_WAVES = 16;
constexpr uint32_t MV_LDS_ROWS = 1024;  // NS * RT partial sums
__host__ __device__ constexpr uint32_t mv_max_threads(int nsb, int d, bool glu) {
  return nsb == 1 && d * (glu ? 2 : 1) <= 8 ? 1024u : 512u;
}

template <class T, int NSB, int D, bool GLU>
__global__ __launch_bounds__(mv_max_threads(NSB, D, GLU)) void k_mv(MV m) {
  __shared__ float vals[MV_LDS_ROWS];  // [NS][RT] partial sums
  __shared__ float vals1[GLU ? MV_LDS_ROWS : 1];
  __shared__ float ssq[MV_MAX_WAVES];
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t s = wv % m.NS, rg = wv / m.NS;
  // segment of this workgroup (uniform)
  uint32_t t = blockIdx.x;
  MVSeg g = m.seg[0];
  if (m.nseg > 1 && t >= m.seg[0].tiles) {
    t -= m.seg[0].tiles;
    g = m.seg[1];
    if (m.nseg > 2 && t >= m.seg[1].tiles) { t -= m.seg[1].tiles; g = m.seg[2]; }
  }
  const Rsrc rw = make_rsrc(g.w, g.bytes);
  const Rsrc rw1 = make_rsrc(GLU ? g.w1 : g.w, g.bytes);
  const uint32_t row0 = t * m.RT;
  const uint32_t part = lane >> m.wshift, cl = lane & (m.Wc - 1);
  // Step i covers rows row0 + rg*P + i*NR*P + part. Chunk of this lane: step + part*C + col,
  // with step = (first row of the step) * C. Rows past the matrix and idle columns load
  // whatever lies there (or zero past the allocation) and their results are dropped.
  const uint32_t rstep = m.NR * m.P, rfirst = rg * m.P;
  uint32_t col[NSB];
  bool valid[NSB];
  typename T::L lc[NSB];
#pragma unroll
  for (int j = 0; j < NSB; j++) {
    const uint32_t c = (s * NSB + j) * m.Wc + cl;
    valid[j] = c < m.C;
    col[j] = valid[j] ? c : 0;
    lc[j] = T::lane(col[j], part * m.C + col[j]);
  }
  typename T::W buf[D][NSB], buf1[GLU ? D : 1][NSB];
  auto issue = [&](int slot, uint32_t i) {
    const uint32_t step = (row0 + rfirst + i * rstep) * m.C;
#pragma unroll
    for (int j = 0; j < NSB; j++) {
      buf[slot][j] = T::load(rw, g.nbt, step, lc[j]);
      if (GLU) buf1[slot][j] = T::load(rw1, g.nbt, step, lc[j]);
    }
  };
  // weight loads first; the activation digits come from L2 while they are in flight
#pragma unroll
  for (int d = 0; d < D; d++) issue(d, d);
  XS<T::N> xs[NSB];
#pragma unroll
  for (int j = 0; j < NSB; j++) {
    if (valid[j]) load_xs<T::N>(m.x, col[j], xs[j]);
    else xs[j] = XS<T::N>{};
  }
  auto step = [&](int slot, uint32_t i) {
    float acc = 0.f, acc1 = 0.f;
#pragma unroll
    for (int j = 0; j < NSB; j++) {
      const float v = T::dot(buf[slot][j], lc[j], xs[j]);
      acc += valid[j] ? v : 0.f;
      if (GLU) {
        const float v1 = T::dot(buf1[slot][j], lc[j], xs[j]);
        acc1 += valid[j] ? v1 : 0.f;
      }
    }
    acc = seg_sum(acc, m.Wc);
    if (GLU) acc1 = seg_sum(acc1, m.Wc);
    if (cl == m.Wc - 1) {
      const uint32_t r = rfirst + part + i * rstep;
      vals[s * m.RT + r] = acc;
      if (GLU) vals1[s * m.RT + r] = acc1;
    }
  };
  // sliding window: ITER is a multiple of D
  uint32_t i0 = 0;
  for (; i0 + D < m.ITER; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      step(d, i0 + d);
      issue(d, i0 + D + d);
    }
  }
#pragma unroll
  for (int d = 0; d < D; d++) step(d, i0 + d);
  if (m.x.normed && rg == 0) {
    // every chunk column once: the lanes of row part 0 of the first row group
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NSB; j++) ss += xs[j].ss;
    ss = wave_sum(part == 0 ? ss : 0.f);
    if (lane == 0) ssq[s] = ss;
  }
  __syncthreads();
  if (threadIdx.x >= ((m.RT + 63) & ~63u)) return;
  float xm = 1.f;
  if (m.x.normed) {
    float tot = 0.f;
    for (uint32_t k = 0; k < m.NS; k++) tot += ssq[k];
    xm = 1.f / sqrtf(tot / (float)m.x.len + m.x.eps);
  }
  const uint32_t r = threadIdx.x;
  const bool inside = r < m.RT && row0 + r < g.rows;
  float v = 0.f, v1 = 0.f;
  if (r < m.RT) {
    for (uint32_t k = 0; k < m.NS; k++) { v += vals[k * m.RT + r]; if (GLU) v1 += vals1[k * m.RT + r]; }
  }
  finish_row(m, g, row0 + r, inside, v * xm, v1 * xm);
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

static uint32_t chunk_of(int type) { return type == Q8_0 ? 16 : 32; }

bool mv_supported(const Matrix &w) {
  if (w.layout != LAYOUT_PLANAR || !w.cols || !w.rows) return false;
  if (w.type == Q4_K || w.type == Q6_K) return w.cols % 256 == 0;
  if (w.type == Q8_0) return w.cols % 32 == 0;
  return false;
}

// The launch shape, searched over the K split (Wc lanes x NSB chunks per lane, NS slices)
// and the rows (NR groups of ITER steps, ITER a multiple of the pipeline depth D). The cost
// is the lane-steps the busiest CU streams (whole rounds of CU-count tiles), stretched when
// a CU holds less than ~48 KB of loads in flight, when the pipeline is shallower than the
// budget allows, and by the per-wavefront activation loads.
MVPlan mv_plan(const Matrix &w, const uint32_t *rows, uint32_t n, bool glu, bool quantized_out) {
  MVPlan best_p{};
  const uint32_t C = w.cols / chunk_of(w.type);
  const uint32_t cus = (uint32_t)device_cu_count();
  static const int env_wc = getenv("WGD_MV_WC") ? atoi(getenv("WGD_MV_WC")) : 0;
  static const int env_nsb = getenv("WGD_MV_NSB") ? atoi(getenv("WGD_MV_NSB")) : 0;
  static const int env_iter = getenv("WGD_MV_ITER") ? atoi(getenv("WGD_MV_ITER")) : 0;
  static const int env_nr = getenv("WGD_MV_NR") ? atoi(getenv("WGD_MV_NR")) : 0;
  double best_cost = 1e30;
  for (uint32_t wc : {64u, 32u, 16u}) {
    if (env_wc && (int)wc != env_wc) continue;
    for (uint32_t nsb : {1u, 2u}) {
      if (env_nsb && (int)nsb != env_nsb) continue;
      MVPlan p{};
      p.C = C; p.Wc = wc; p.NSB = nsb; p.P = 64 / wc;
      p.NS = (C + wc * nsb - 1) / (wc * nsb);
      const uint32_t waste = p.NS * wc * nsb - C;
      if (p.NS > MV_MAX_WAVES) continue;
      // D row steps x NSB chunks (x2 for gated pairs) of loads in flight, up to 16
      const uint32_t per_step = nsb * (glu ? 2 : 1);
      const uint32_t dmax = per_step >= 4 ? 4 : 8;
      for (uint32_t nr = 1; nr * p.NS <= MV_MAX_WAVES; nr++) {
        if (env_nr && (int)nr != env_nr) continue;
        for (uint32_t d = dmax; d >= 1; d /= 2) {
          if (64 * nr * p.NS > mv_max_threads((int)nsb, (int)d, glu)) continue;
          for (uint32_t iter = d; iter <= 64 * d; iter += d) {
            if (env_iter && (int)iter != env_iter) continue;
            const uint32_t rt = nr * p.P * iter;
            if (rt > 64 * nr * p.NS || p.NS * rt > MV_LDS_ROWS) break;  // one epilogue thread per row
            if (quantized_out && rt % 16) continue;
            uint32_t tiles = 0;
            for (uint32_t i = 0; i < n; i++) tiles += (rows[i] + rt - 1) / rt;
            const uint32_t rounds = (tiles + cus - 1) / cus;
            // Little's law: a CU streams at full share with ~48 KB of loads in flight; each
            // chunk load of a wavefront is 1 KB (64 lanes x 16 B)
            const double resident = tiles >= 2 * cus ? 2.0 : tiles > cus ? (double)tiles / cus : 1.0;
            const double inflight = (double)(nr * p.NS) * (iter < d ? iter : d) * per_step * resident;
            double cost = (double)rounds * rt * (1.0 + (double)waste / C);  // lane-steps through the busiest CU
            if (inflight < 48.0) cost *= 48.0 / inflight;
            if (iter > d) cost *= 1.0 + 0.25 * (dmax / d - 1);           // fewer loads per round trip
            cost *= 1.0 + 0.5 / iter;  // activation loads of a wavefront, amortised over its row steps
            if (cost < best_cost) {
              best_cost = cost;
              p.NR = nr; p.ITER = iter; p.D = d; p.RT = rt; p.tiles = tiles; p.threads = 64 * nr * p.NS;
              best_p = p;
            }
            if (tiles <= cus) break;  // more steps only lengthen the tile
          }
          if (env_iter) break;
        }
      }
    }
  }
  return best_p;
}

template <class T, bool GLU>
static hipError_t launch_t(hipStream_t s, const MV &m, const MVPlan &p) {
  const dim3 grid(p.tiles), block(p.threads);
#define WGD_MV_CASE(NSB_, D_) \
  if (p.NSB == NSB_ && p.D == D_) { hipLaunchKernelGGL((k_mv<T, NSB_, D_, GLU>), grid, block, 0, s, m); return hipGetLastError(); }
  WGD_MV_CASE(1, 8) WGD_MV_CASE(1, 4) WGD_MV_CASE(1, 2) WGD_MV_CASE(1, 1)
  WGD_MV_CASE(2, 4) WGD_MV_CASE(2, 2) WGD_MV_CASE(2, 1)
  if constexpr (!GLU) { WGD_MV_CASE(2, 8) }  // a gated pair keeps at most 16 chunk loads in flight
#undef WGD_MV_CASE
  return hipErrorInvalidValue;
}

hipError_t mv(hipStream_t s, const MVTarget *t, uint32_t n, const QXView &x, int epi, const MVOut *out) {
  if (n < 1 || n > (uint32_t)MV_MAX_SEGS) return hipErrorInvalidValue;
  const Matrix &w0 = *t[0].w;
  const bool glu = t[0].w1 != nullptr;
  const bool qout = out && out->q.d0;
  if (qout && n != 1) return hipErrorInvalidValue;
  if ((epi == MV_SILU || epi == MV_GELU) != glu) return hipErrorInvalidValue;
  uint32_t rows[MV_MAX_SEGS];
  for (uint32_t i = 0; i < n; i++) {
    const Matrix &w = *t[i].w;
    if (!mv_supported(w) || w.type != w0.type || w.cols != w0.cols || !t[i].y) return hipErrorInvalidValue;
    if ((t[i].w1 != nullptr) != glu) return hipErrorInvalidValue;
    if (glu) {
      const Matrix &w1 = *t[i].w1;
      if (w1.type != w.type || w1.layout != w.layout || w1.cols != w.cols || w1.rows != w.rows) return hipErrorInvalidValue;
    }
    rows[i] = w.rows;
  }
  const MVPlan p = mv_plan(w0, rows, n, glu, qout);
  if (!p.RT || p.threads != 64 * p.NS * p.NR || p.threads > mv_max_threads((int)p.NSB, (int)p.D, glu) ||
      p.RT > p.threads || p.ITER % p.D || p.NS * p.RT > MV_LDS_ROWS || (p.NSB != 1 && p.NSB != 2) || !p.Wc ||
      64 % p.Wc || (qout && p.RT % 16))
    return hipErrorInvalidValue;
  MV m{};
  m.nseg = n;
  for (uint32_t i = 0; i < n; i++) {
    const Matrix &w = *t[i].w;
    MVSeg &g = m.seg[i];
    g.w = w.data; g.w1 = glu ? t[i].w1->data : nullptr;
    const uint64_t nbt = (uint64_t)(w.cols / block_size(w.type)) * w.rows, bytes = nbt * block_bytes(w.type);
    if (bytes >= (1ull << 32)) return hipErrorInvalidValue;  // 32-bit buffer offsets
    g.nbt = (uint32_t)nbt;
    g.bytes = (uint32_t)bytes;
    g.y = t[i].y; g.bias = t[i].bias;
    g.rows = w.rows;
    g.tiles = (w.rows + p.RT - 1) / p.RT;
  }
  m.x = x;
  m.C = p.C; m.Wc = p.Wc; m.P = p.P; m.NS = p.NS; m.NR = p.NR; m.ITER = p.ITER; m.RT = p.RT;
  m.wshift = 0;
  while ((1u << m.wshift) < p.Wc) m.wshift++;
  m.epi = epi;
  m.oq = QXOut{};
  m.oq_norm = nullptr;
  if (qout) { m.oq = out->q; m.oq_norm = out->norm_w; }
  switch (w0.type) {
    case Q4_K: return glu ? launch_t<CQ4K, true>(s, m, p) : launch_t<CQ4K, false>(s, m, p);
    case Q6_K: return glu ? launch_t<CQ6K, true>(s, m, p) : launch_t<CQ6K, false>(s, m, p);
    case Q8_0: return glu ? launch_t<CQ80, true>(s, m, p) : launch_t<CQ80, false>(s, m, p);
  }
  return hipErrorInvalidValue;
}

}  // namespace wgd
