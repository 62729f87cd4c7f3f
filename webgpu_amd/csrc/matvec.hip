// matvec.hip — decode dequant-matvec (batch 1) for gfx950 on integer dot products.
//
// Replaces matmulShader (src/core/shaders.ts:39-54) for one activation row. The reference
// decodes every weight to f32 and multiplies by an f32 activation. Here the activation row
// is first quantized ("QX" format): per 32-element block a scale s = max|x| / 127 and three
// signed base-254 digits per element, x = s * (d0 + d1/254 + d2/254^2) (error <= 6.1e-8 * max|x|,
// i.e. f32-level). Each weight block is then consumed in its raw form: 4-bit (Q4_K), 6-bit
// (Q6_K) or 8-bit (Q8_0) quants are masked into bytes and multiplied with the digits by
// v_dot4_i32_i8, four products per instruction, exact in int32. The block scales are applied
// once per 16/32-element group; the Q4_K minimum and the Q6_K offset use exact f32 sums of x.
//
// Work split: a workgroup owns RT rows; its NS wavefronts split K into slices of W units
// (a unit is the 64 (Q4_K, Q6_K) or 32 (Q8_0) weights one lane handles per row), load the
// activation digits of their slice once and stream the RT rows, W lanes per row, P = 64/W
// rows per pass. The slices are summed through LDS in slice order (deterministic) and wave
// 0 runs the epilogue: store, residual add, or the gated SwiGLU/GeGLU of a gate/up pair,
// optionally re-quantizing the result (times the next RMSNorm weight) into the QX buffer of
// the next matvec. Nothing synchronizes across workgroups inside a launch: on MI355X each
// XCD has its own L2, and device-scope fences write back and invalidate it.
#include <cstdlib>

#include "internal.h"
#include "decode.h"
#include "matvec.h"

namespace wgd {

// ------------------------------------------------------------------ quantization helpers

// Quantizes one value per lane in aligned 32-lane groups. Returns the three digits packed in
// the low 24 bits; the block scale (max|v| / 127) is returned through `scale`.
__device__ __forceinline__ void quant_lane32(float v, float &scale, int &d0, int &d1, int &d2) {
  float a = fabsf(v);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
  scale = a * (1.f / 127.f);
  float u = a > 0.f ? v * (127.f / a) : 0.f;
  float r0 = rintf(u);
  r0 = fminf(fmaxf(r0, -127.f), 127.f);
  float t = (u - r0) * 254.f;
  float r1 = fminf(fmaxf(rintf(t), -127.f), 127.f);
  float t2 = (t - r1) * 254.f;
  float r2 = fminf(fmaxf(rintf(t2), -127.f), 127.f);
  d0 = (int)r0; d1 = (int)r1; d2 = (int)r2;
}

// Writes element `i` of a QX vector (value v already multiplied by any norm weight), with the
// block scale and the 16-element sums. Lanes must hold 32 consecutive aligned elements.
__device__ __forceinline__ void qx_store(const QXOut &q, uint32_t i, float v, bool live) {
  float sc; int d0, d1, d2;
  quant_lane32(live ? v : 0.f, sc, d0, d1, d2);
  float s16 = live ? v : 0.f;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) s16 += __shfl_xor(s16, o, 64);
  if (live) {
    q.d0[i] = (int8_t)d0; q.d1[i] = (int8_t)d1; q.d2[i] = (int8_t)d2;
    if ((i & 31) == 0) q.scale[i >> 5] = sc;
    if ((i & 15) == 0) q.sum16[i >> 4] = s16;
  }
}

// Standalone quantization of x (length K), optionally as x * w with the RMSNorm inverse
// left to the consumer: one workgroup per 256 elements, each leaving its sum of squares.
__global__ __launch_bounds__(256) void k_quantize(const float *x, uint32_t K, const float *w, float eps, QXOut q) {
  __shared__ float red[4];
  const uint32_t tid = threadIdx.x, i = blockIdx.x * 256 + tid;
  const bool live = i < K;
  const float v = live ? x[i] : 0.f;
  qx_store(q, i, (live && w) ? v * w[i] : v, live);
  if (w) {
    float ss = wave_sum(v * v);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    if (tid == 0) q.sq[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
  }
  if (blockIdx.x == 0 && tid == 0) {
    q.hdr->mul = 1.f;
    q.hdr->ntiles = w ? gridDim.x : 0;
    q.hdr->len = K;
    q.hdr->eps = eps;
  }
}

// ------------------------------------------------------------------ unit kernels

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Activation digits used by the matvec. Two (x within 1.6e-5 * max|x| of its 32-element block)
// exceed a 1e-3 relative logits bound at the 8B decoder shape; three are f32-level.
constexpr int DIG = 3;

// Streaming (non-temporal) loads of weight bytes, which are read once per token.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 nt16(const uint8_t *p) {
  u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 nt8(const uint8_t *p) {
  u32x2_t v = __builtin_nontemporal_load((const u32x2_t *)p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t nt2(const uint8_t *p) { return __builtin_nontemporal_load((const uint16_t *)p); }

// Activation digits for one unit, plus block scales and sums.
template <int N> struct XD {
  int d[DIG][N / 4]; // packed int8 digits
  float s[N / 16];   // scale per 16 elements (the 32-block scale, repeated)
  float sum[N / 16]; // exact sums per 16 elements
};

__device__ __forceinline__ void load16(const int8_t *p, int *dst) {
  int4 v = *(const int4 *)p;
  dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
}

__device__ __forceinline__ float combine(const int *sd) {
  float r = (float)sd[0];
  if (DIG > 1) r += (float)sd[1] * (1.f / 254.f);
  if (DIG > 2) r += (float)sd[2] * (1.f / 64516.f);
  return r;
}

struct MQ4K {
  static constexpr int UNIT = 64;
  // Unit u = (block u/4, 32-byte quant group u%4): elements [64u, 64u + 64) — the low nibbles
  // of the group are sub-block 2g, the high nibbles sub-block 2g+1.
  static __device__ __forceinline__ void load_x(const QXView &x, uint32_t u, XD<64> &xd) {
#pragma unroll
    for (int d = 0; d < DIG; d++)
#pragma unroll
      for (int c = 0; c < 4; c++) load16(x.d[d] + 64 * u + 16 * c, &xd.d[d][4 * c]);
#pragma unroll
    for (int c = 0; c < 4; c++) { xd.s[c] = x.scale[2 * u + c / 2]; xd.sum[c] = x.sum16[4 * u + c]; }
  }
  struct Raw { uint4 h, a, b; };
  // Planar layout: the 128 quant bytes of every block in one plane, the 16-byte headers
  // (d, dmin, packed scales) in another, so consecutive lanes read consecutive bytes.
  static __device__ __forceinline__ Raw load_from(const uint8_t *w, const MV &m, uint32_t row, uint32_t u) {
    Raw r;
    const uint32_t g = u & 3;
    if (m.layout == LAYOUT_PLANAR) {
      Q4Planes p = q4_planes(m.nbt);
      const uint64_t bi = (uint64_t)row * m.bpr + (u >> 2);
      r.h = nt16(w + p.hdr + bi * 16);
      r.a = nt16(w + p.qs + bi * 128 + 32 * g);
      r.b = nt16(w + p.qs + bi * 128 + 32 * g + 16);
    } else {
      const uint8_t *blk = w + (uint64_t)row * m.rb + (uint64_t)(u >> 2) * 144;
      r.h = *(const uint4 *)blk;
      r.a = *(const uint4 *)(blk + 16 + 32 * g);
      r.b = *(const uint4 *)(blk + 32 + 32 * g);
    }
    return r;
  }
  static __device__ __forceinline__ Raw load(const MV &m, uint32_t row, uint32_t u) { return load_from(m.w, m, row, u); }
  static __device__ __forceinline__ Raw load1(const MV &m, uint32_t row, uint32_t u) { return load_from(m.w1, m, row, u); }
  static __device__ __forceinline__ float dot(const Raw &r, uint32_t u, const XD<64> &xd) {
    const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    int lo[DIG] = {}, hi[DIG] = {};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      int l = (int)(q[k] & 0x0F0F0F0Fu), h = (int)((q[k] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int d = 0; d < DIG; d++) { lo[d] = dot4(l, xd.d[d][k], lo[d]); hi[d] = dot4(h, xd.d[d][8 + k], hi[d]); }
    }
    // scale/min of sub-blocks 2g, 2g+1 (quant.ts:15-16): bytes 2g&3, +1 of the packed scales
    const uint32_t g = u & 3, sh = 16 * (g & 1);
    const uint32_t A = r.h.y >> sh, B = r.h.z >> sh, C = r.h.w >> sh;
    uint32_t scp, mnp;
    if (g < 2) { scp = A & 0x3F3Fu; mnp = B & 0x3F3Fu; }
    else { scp = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u); mnp = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u); }
    const float d = __half2float(__ushort_as_half((unsigned short)(r.h.x & 0xFFFFu)));
    const float dm = __half2float(__ushort_as_half((unsigned short)(r.h.x >> 16)));
    const float qx0 = xd.s[0] * combine(lo);
    const float qx1 = xd.s[2] * combine(hi);
    const float sc0 = (float)(scp & 0xFFu), sc1 = (float)(scp >> 8);
    const float mn0 = (float)(mnp & 0xFFu), mn1 = (float)(mnp >> 8);
    return d * (sc0 * qx0 + sc1 * qx1) - dm * (mn0 * (xd.sum[0] + xd.sum[1]) + mn1 * (xd.sum[2] + xd.sum[3]));
  }
};

struct MQ6K {
  static constexpr int UNIT = 64;
  // Unit u = (block u/4, 128-element half (u/2)&1, 16-lane half u&1): for quarter t the 16
  // elements b*256 + seg*128 + 32t + 16h ... +16 (quant.ts:21-27).
  static __device__ __forceinline__ uint32_t base(uint32_t u, int t) {
    return (u >> 2) * 256 + ((u >> 1) & 1) * 128 + 32 * t + 16 * (u & 1);
  }
  static __device__ __forceinline__ void load_x(const QXView &x, uint32_t u, XD<64> &xd) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
      uint32_t b = base(u, t);
#pragma unroll
      for (int d = 0; d < DIG; d++) load16(x.d[d] + b, &xd.d[d][4 * t]);
      xd.s[t] = x.scale[b >> 5];
      xd.sum[t] = x.sum16[b >> 4];
    }
  }
  struct Raw { uint4 a, b, h; uint2 s; uint32_t d; };
  static __device__ __forceinline__ Raw load_from(const uint8_t *w, const MV &m, uint32_t row, uint32_t u) {
    Q6Planes p = q6_planes(m.nbt);
    uint64_t bi = (uint64_t)row * m.bpr + (u >> 2);
    uint32_t seg = (u >> 1) & 1, h = u & 1;
    const uint8_t *ql = w + p.ql + bi * 128 + seg * 64 + 16 * h;
    Raw r;
    r.a = nt16(ql);
    r.b = nt16(ql + 32);
    r.h = nt16(w + p.qh + bi * 64 + seg * 32 + 16 * h);
    r.s = nt8(w + p.sc + bi * 16 + seg * 8);
    r.d = nt2(w + p.d + bi * 2);
    return r;
  }
  static __device__ __forceinline__ Raw load(const MV &m, uint32_t row, uint32_t u) { return load_from(m.w, m, row, u); }
  static __device__ __forceinline__ Raw load1(const MV &m, uint32_t row, uint32_t u) { return load_from(m.w1, m, row, u); }
  static __device__ __forceinline__ float dot(const Raw &r, uint32_t u, const XD<64> &xd) {
    const uint32_t h = u & 1;
    const uint32_t qa[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, qb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    const uint32_t qh[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      int s[DIG] = {};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t src = (t & 1) ? qb[k] : qa[k];
        uint32_t lo = (t & 2) ? ((src >> 4) & 0x0F0F0F0Fu) : (src & 0x0F0F0F0Fu);
        int q = (int)(lo | (((qh[k] >> (2 * t)) & 0x03030303u) << 4));
#pragma unroll
        for (int d = 0; d < DIG; d++) s[d] = dot4(q, xd.d[d][4 * t + k], s[d]);
      }
      const uint32_t sw = (t < 2) ? r.s.x : r.s.y;
      const float sc = (float)(int8_t)((sw >> (8 * ((2 * t + h) & 3))) & 0xFFu);
      acc += sc * (xd.s[t] * combine(s) - 32.f * xd.sum[t]);
    }
    return __half2float(__ushort_as_half((unsigned short)r.d)) * acc;
  }
};

struct MQ80 {
  static constexpr int UNIT = 32;
  static __device__ __forceinline__ void load_x(const QXView &x, uint32_t u, XD<32> &xd) {
#pragma unroll
    for (int d = 0; d < DIG; d++) { load16(x.d[d] + 32 * u, &xd.d[d][0]); load16(x.d[d] + 32 * u + 16, &xd.d[d][4]); }
    xd.s[0] = xd.s[1] = x.scale[u];
    xd.sum[0] = xd.sum[1] = 0.f;
  }
  struct Raw { uint4 a, b; uint32_t d; };
  static __device__ __forceinline__ Raw load_from(const uint8_t *w, const MV &m, uint32_t row, uint32_t u) {
    Q8Planes p = q8_planes(m.nbt);
    uint64_t bi = (uint64_t)row * m.bpr + u;
    Raw r;
    r.a = nt16(w + p.qs + bi * 32);
    r.b = nt16(w + p.qs + bi * 32 + 16);
    r.d = nt2(w + p.d + bi * 2);
    return r;
  }
  static __device__ __forceinline__ Raw load(const MV &m, uint32_t row, uint32_t u) { return load_from(m.w, m, row, u); }
  static __device__ __forceinline__ Raw load1(const MV &m, uint32_t row, uint32_t u) { return load_from(m.w1, m, row, u); }
  static __device__ __forceinline__ float dot(const Raw &r, uint32_t u, const XD<32> &xd) {
    const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    int s[DIG] = {};
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
      for (int d = 0; d < DIG; d++) s[d] = dot4((int)q[k], xd.d[d][k], s[d]);
    return __half2float(__ushort_as_half((unsigned short)r.d)) * xd.s[0] * combine(s);
  }
};

// ------------------------------------------------------------------ the tile kernel

__device__ __forceinline__ float gelu_tanh_mv(float g) {
  return 0.5f * g * (1.f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g)));
}

__device__ __forceinline__ float seg_sum(float v, uint32_t width) {
  for (uint32_t o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// The activation multiplier: 1, a stored value, or the RMSNorm inverse reduced from the
// producer's per-tile sums of squares (tile order, deterministic). Wave-uniform.
__device__ __forceinline__ float qx_mul(const QXView &x) {
  const uint32_t n = x.hdr->ntiles;
  if (n == 0) return x.hdr->mul;
  float t = 0.f;
  for (uint32_t i = threadIdx.x & 63; i < n; i += 64) t += x.sq[i];
  t = wave_sum(t);
  return 1.f / sqrtf(t / (float)x.hdr->len + x.hdr->eps);
}

// Epilogue of one row tile in wave 0: lane i < RT holds row rt * RT + i.
__device__ __forceinline__ void finish_tile(const MV &m, uint32_t rt, float v, float u, float xm) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t row = rt * m.RT + lane;
  const bool live = lane < m.RT && row < m.rows;
  v *= xm; u *= xm;
  float out = 0.f;
  if (live) {
    float *dst = m.y + m.row_base + row;
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
    qx_store(m.oq, row, out * wn, live);
    if (m.oq_norm) {
      const float sq = wave_sum(live ? out * out : 0.f);
      if (lane == 0) m.oq.sq[rt] = sq;
    }
    if (rt == 0 && lane == 0) {
      m.oq.hdr->mul = 1.f;
      m.oq.hdr->ntiles = m.oq_norm ? m.tiles_rows : 0;
      m.oq.hdr->len = m.rows;
      m.oq.hdr->eps = m.oq_eps;
    }
  }
}

// One workgroup per row tile; wave s handles K-slice s. NT = max threads of the variant.
// PIPE = false issues the loads of R rows at once per round (a tile of J <= R rows per lane
// segment is one round-trip); PIPE = true keeps the next R rows in flight while R compute.
template <class T, int R, bool GLU, int NT, bool PIPE>
__global__ __launch_bounds__(NT) void k_mv(MV m) {
  __shared__ float vals[16][64], vals1[16][64];
  __shared__ float xmul;
  const uint32_t lane = threadIdx.x & 63, s = threadIdx.x >> 6;
  const uint32_t rt = blockIdx.x;
  const uint32_t seg = lane / m.W, ul = lane % m.W, u = s * m.W + ul;
  const bool valid = u < m.U;
  XD<T::UNIT> xd;
  if (valid) T::load_x(m.x, u, xd);
  else xd = XD<T::UNIT>{};  // zero digits, scales and sums: an idle lane's dot is exactly 0
  if (s == 0) {
    const float xm = qx_mul(m.x);
    if (lane == 0) xmul = xm;
  }
  const uint32_t row0 = rt * m.RT;
  const uint32_t J = m.RT / m.P;
  // Rows of this lane segment: row0 + seg + P*j, j < J. Out-of-range rows read a clamped
  // valid row (no divergent loads) and their results are dropped.
  auto row_of = [&](uint32_t j) -> uint32_t {
    const uint32_t r = row0 + seg + m.P * j;
    return r < m.rows ? r : m.rows - 1;
  };
  const uint32_t uu = valid ? u : 0;
  // Two-stage pipeline: the loads of the next R rows are in flight while R rows compute.
  typename T::Raw cur[R], cur1[R], nxt[R], nxt1[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    cur[r] = T::load(m, row_of(r < (int)J ? r : 0), uu);
    if (GLU) cur1[r] = T::load1(m, row_of(r < (int)J ? r : 0), uu);
  }
  for (uint32_t j0 = 0; j0 < J; j0 += R) {
    const bool more = j0 + R < J;
    if (!PIPE && j0 > 0) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t j = j0 + r < J ? j0 + r : j0;
        cur[r] = T::load(m, row_of(j), uu);
        if (GLU) cur1[r] = T::load1(m, row_of(j), uu);
      }
    }
    if (PIPE && more) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t j = j0 + R + r < J ? j0 + R + r : j0 + R;
        nxt[r] = T::load(m, row_of(j), uu);
        if (GLU) nxt1[r] = T::load1(m, row_of(j), uu);
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      float acc = T::dot(cur[r], uu, xd);
      float acc1 = GLU ? T::dot(cur1[r], uu, xd) : 0.f;
      acc = seg_sum(acc, m.W);
      if (GLU) acc1 = seg_sum(acc1, m.W);
      const uint32_t li = seg + m.P * (j0 + r);
      if (ul == 0 && j0 + r < J) { vals[s][li] = acc; if (GLU) vals1[s][li] = acc1; }
    }
    if (PIPE && more) {
#pragma unroll
      for (int r = 0; r < R; r++) { cur[r] = nxt[r]; if (GLU) cur1[r] = nxt1[r]; }
    }
  }
  __syncthreads();
  if (s != 0) return;
  float v = 0.f, v1 = 0.f;
  if (lane < m.RT) {
    for (uint32_t k = 0; k < m.NS; k++) { v += vals[k][lane]; if (GLU) v1 += vals1[k][lane]; }
  }
  finish_tile(m, rt, v, v1, xmul);
}

// ------------------------------------------------------------------ host side

uint64_t qx_bytes(uint32_t K) {
  uint64_t kp = (K + 63) / 64 * 64;
  return 3 * kp + 4 * (kp / 32) + 4 * (kp / 16) + sizeof(QXHeader) + 4 * QX_MAX_TILES;
}

QXOut qx_view(void *base, uint32_t K) {
  uint64_t kp = (K + 63) / 64 * 64;
  uint8_t *p = (uint8_t *)base;
  QXOut q;
  q.d0 = (int8_t *)p; q.d1 = (int8_t *)(p + kp); q.d2 = (int8_t *)(p + 2 * kp);
  q.scale = (float *)(p + 3 * kp);
  q.sum16 = q.scale + kp / 32;
  q.hdr = (QXHeader *)(q.sum16 + kp / 16);
  q.sq = (float *)(q.hdr + 1);
  return q;
}

QXView qx_const(const QXOut &q) {
  QXView v;
  v.d[0] = q.d0; v.d[1] = q.d1; v.d[2] = q.d2; v.scale = q.scale; v.sum16 = q.sum16; v.hdr = q.hdr; v.sq = q.sq;
  return v;
}

hipError_t quantize(hipStream_t s, const float *x, uint32_t K, const float *norm_w, float eps, const QXOut &q) {
  const uint32_t blocks = (K + 255) / 256;
  if (!K || blocks > QX_MAX_TILES) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_quantize, dim3(blocks), dim3(256), 0, s, x, K, norm_w, eps, q);
  return hipGetLastError();
}

static uint32_t unit_of(int type) { return type == Q8_0 ? 32 : 64; }

bool mv_supported(const Matrix &w) {
  if (w.type == Q4_K) return w.cols % 256 == 0;
  if (w.type == Q6_K) return w.layout == LAYOUT_PLANAR && w.cols % 256 == 0;
  if (w.type == Q8_0) return w.layout == LAYOUT_PLANAR && w.cols % 32 == 0;
  return false;
}

// Tiling: the widest slice (fewest wavefronts per row tile) whose idle lanes stay under 1/7
// and that still yields enough wavefronts to cover the chip; RT is the row-tile height.
MVPlan mv_plan(const Matrix &w, bool quantized_out) {
  MVPlan p;
  const uint32_t U = w.cols / unit_of(w.type);
  const uint32_t target = (uint32_t)device_cu_count() * 8;
  const uint32_t widths[5] = {64, 32, 16, 8, 4};
  static const int env_w = getenv("WGD_MV_W") ? atoi(getenv("WGD_MV_W")) : 0;
  static const int env_rt = getenv("WGD_MV_RT") ? atoi(getenv("WGD_MV_RT")) : 0;
  auto rt_of = [&](uint32_t W, uint32_t NS) -> uint32_t {
    const uint32_t P = 64 / W;
    if (quantized_out) return 32;
    if (env_rt >= (int)P && env_rt <= 64 && env_rt % P == 0) return (uint32_t)env_rt;
    // Rows per tile: at least one pass per lane segment, at most 64; smaller tiles when the
    // matrix has too few rows to give every CU several wavefronts.
    uint32_t rt = 64;
    while (rt > P * 2 && NS * ((w.rows + rt - 1) / rt) < target) rt /= 2;
    return rt < P ? P : rt;
  };
  int pick = -1, fallback = 0;
  uint32_t least_waste = 0xFFFFFFFFu;
  for (int i = 0; i < 5; i++) {
    const uint32_t W = widths[i], NS = (U + W - 1) / W, waste = NS * W - U;
    if (env_w && (int)W != env_w) continue;
    if (NS > 8) continue;
    if (waste < least_waste) { least_waste = waste; fallback = i; }
    if (waste * 7 > U) continue;
    const uint32_t rt = rt_of(W, NS), waves = NS * ((w.rows + rt - 1) / rt);
    pick = i;
    if (waves >= target) break;
  }
  if (pick < 0) pick = fallback;
  p.W = widths[pick];
  p.P = 64 / p.W;
  p.NS = (U + p.W - 1) / p.W;
  p.RT = rt_of(p.W, p.NS);
  p.tiles_rows = (w.rows + p.RT - 1) / p.RT;
  p.U = U;
  static const int env_r = getenv("WGD_MV_R") ? atoi(getenv("WGD_MV_R")) : 0;
  p.R = env_r > 0 ? (uint32_t)env_r : 0;
  return p;
}

template <class T>
static hipError_t launch_t(hipStream_t s, const MV &m, bool glu, uint32_t R) {
  const dim3 grid(m.tiles_rows), block(64 * m.NS);
  const uint32_t J = m.RT / m.P;
  // R == 0 (default): one round-trip per tile when its rows fit the register budget.
  if (glu) {
    if ((R == 0 && J <= 4) || R == 4) hipLaunchKernelGGL((k_mv<T, 4, true, 512, false>), grid, block, 0, s, m);
    else if (R == 1) hipLaunchKernelGGL((k_mv<T, 1, true, 512, true>), grid, block, 0, s, m);
    else hipLaunchKernelGGL((k_mv<T, 2, true, 512, true>), grid, block, 0, s, m);
  } else {
    if ((R == 0 && J <= 4) || R == 4) hipLaunchKernelGGL((k_mv<T, 4, false, 512, false>), grid, block, 0, s, m);
    else if ((R == 0 && J <= 8) || R == 8) hipLaunchKernelGGL((k_mv<T, 8, false, 512, false>), grid, block, 0, s, m);
    else hipLaunchKernelGGL((k_mv<T, 2, false, 512, true>), grid, block, 0, s, m);
  }
  return hipGetLastError();
}

hipError_t mv(hipStream_t s, const Matrix &w, const Matrix *w1, const QXView &x, float *y, uint32_t row_base,
              int epi, const MVOut *out) {
  if (!mv_supported(w)) return hipErrorInvalidValue;
  const bool glu = w1 != nullptr;
  if (glu && (w1->type != w.type || w1->layout != w.layout || w1->cols != w.cols || w1->rows != w.rows))
    return hipErrorInvalidValue;
  const bool qout = out && out->q.d0;
  MVPlan p = mv_plan(w, qout);
  if (p.NS > 8 || p.RT > 64 || (qout && out->norm_w && p.tiles_rows > QX_MAX_TILES)) return hipErrorInvalidValue;
  MV m;
  m.w = w.data; m.w1 = glu ? w1->data : nullptr;
  m.layout = w.layout;
  m.rb = row_bytes(w.type, w.cols);
  m.bpr = w.cols / block_size(w.type);
  m.nbt = (uint64_t)m.bpr * w.rows;
  m.x = x;
  m.cols = w.cols; m.rows = w.rows; m.U = p.U; m.W = p.W; m.P = p.P; m.NS = p.NS; m.RT = p.RT;
  m.tiles_rows = p.tiles_rows;
  m.y = y; m.row_base = row_base; m.epi = epi;
  m.oq = QXOut{};
  m.oq_norm = nullptr; m.oq_eps = 0.f;
  if (qout) { m.oq = out->q; m.oq_norm = out->norm_w; m.oq_eps = out->eps; }
  switch (w.type) {
    case Q4_K: return launch_t<MQ4K>(s, m, glu, p.R);
    case Q6_K: return launch_t<MQ6K>(s, m, glu, p.R);
    case Q8_0: return launch_t<MQ80>(s, m, glu, p.R);
  }
  return hipErrorInvalidValue;
}

}  // namespace wgd
