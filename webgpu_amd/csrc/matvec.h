// matvec.h — quantized-activation format and the decode matvec (matvec.hip).
#pragma once
#include "internal.h"

namespace wgd {

// A quantized activation vector of K elements ("QX", K % 16 == 0): three int8 digit planes
// and, per 16-element block, the f32 scale (max|x| / 127), the exact f32 sum and the f32
// sum of squares of the values before any norm weight. The stored values are x, or x * w
// for an RMSNorm with weight w whose 1/sqrt(mean(x^2) + eps) is still pending: the consumer
// applies it to its dot products after reducing the sums of squares over the whole vector
// inside each workgroup (every workgroup reads all of K), so no launch needs a
// cross-workgroup reduction. 16-element blocks let a producer quantize its output in
// 16-row tiles. Three digits are f32-level; two (x within 1.6e-5 * max|x| of its block)
// exceed a 1e-3 relative logits bound at the 8B decoder shape. Layout in one buffer of
// qx_bytes(K), Kp = K rounded up to 64:
//   d0[Kp] d1[Kp] d2[Kp] | scale[Kp/16] sum[Kp/16] sq[Kp/16]
struct QXOut {
  int8_t *d0 = nullptr, *d1 = nullptr, *d2 = nullptr;
  float *scale = nullptr, *sum = nullptr, *sq = nullptr;
};
struct QXView {
  const int8_t *d[3];
  const float *scale, *sum, *sq;
  uint32_t normed;  // nonzero: the values carry a norm weight; multiplier from sq
  uint32_t len;     // K, the mean's divisor
  float eps;
};
uint64_t qx_bytes(uint32_t K);
QXOut qx_view(void *base, uint32_t K);
QXView qx_const(const QXOut &q, uint32_t K, bool normed, float eps);

#ifdef __HIPCC__
// Max / sum over each aligned 16-lane row of the wavefront, left in every lane of the row:
// DPP quad xor 1, quad xor 2, half-row mirror, row mirror (VALU moves, no LDS round trip).
// Every lane of the row must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  return fmaxf(v, dpp_mov<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  return v + dpp_mov<0x140>(v);
}

// Quantizes one value per lane in aligned 16-lane groups; the block scale is max|v| / 127.
__device__ __forceinline__ void quant_lane16(float v, float &scale, int &d0, int &d1, int &d2) {
  const float a = row16_max(fabsf(v));
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
  const float s16 = row16_sum(live ? v : 0.f), q16 = row16_sum(live ? raw * raw : 0.f);
  if (live) {
    q.d0[i] = (int8_t)d0; q.d1[i] = (int8_t)d1; q.d2[i] = (int8_t)d2;
    if ((i & 15) == 0) { q.scale[i >> 4] = sc; q.sum[i >> 4] = s16; q.sq[i >> 4] = q16; }
  }
}
#endif

// x (length K, K % 16 == 0) -> QX; with norm_w the stored values are x * norm_w.
hipError_t quantize(hipStream_t s, const float *x, uint32_t K, const float *norm_w, const QXOut &q);
// One row: state += RMSNorm(delta) * w (Gemma's post-norms), then the QX of the new state
// times next_w (n % 16 == 0), in one launch.
hipError_t norm_add_quantize(hipStream_t s, const float *delta, const float *w, float *state, uint32_t n, float eps,
                             const float *next_w, const QXOut &q);

enum MVEpilogue : int { MV_STORE = 0, MV_ADD = 1, MV_SILU = 2, MV_GELU = 3 };

// Re-quantization of a matvec's output for the next consumer: the stored vector is
// y * norm_w when norm_w is set (the consumer then applies the RMSNorm multiplier).
struct MVOut {
  QXOut q;
  const float *norm_w = nullptr;
  uint64_t *arg_part = nullptr;  // argmax key (first index of the finite max) per epilogue wavefront:
                                 // mv_arg_entries() of them
};

// One matrix of a launch. Several matrices that read the same activation (the Q, K and V
// projections) run in one launch, one row-tile range each: of one type, or Q4_K and Q6_K.
struct MVTarget {
  const Matrix *w = nullptr;
  const Matrix *w1 = nullptr;  // the up matrix of a gated pair (MV_SILU / MV_GELU)
  float *y = nullptr;
  const float *bias = nullptr;
};

// Launch shape. A wavefront computes 16 rows x 4 chunk columns per MFMA "unit" (lane = row
// r % 16, column group g); a workgroup owns RT = 16 * NR * ITER rows, its NS x NR wavefronts
// split K into NS slices of NSB units (4 * NSB chunk columns) and the row tiles into NR
// groups of ITER steps; each wavefront runs its U = ITER * NSB units with DU in flight.
struct MVPlan { uint32_t C, NS, NSB, NR, ITER, DU, RT, tiles, threads, lds; };

constexpr int MV_MAX_SEGS = 3;
struct MVSeg {
  const uint8_t *w, *w1;
  uint32_t bytes;      // allocation size (buffer range)
  uint32_t nbp;        // blocks of the padded matrix (plane offsets)
  uint32_t bpr;        // blocks per row
  uint32_t rows, tiles;
  uint32_t kind;       // chunk type: 0 the launch's first, 1 the other K-quant
  float *y;
  const float *bias;
};
struct MV {
  MVSeg seg[MV_MAX_SEGS];
  uint32_t nseg;
  QXView x;
  uint32_t C, ke;      // chunk columns; staged activation elements (NS * NSB * 4 chunks)
  uint32_t NS, NSB, NR, ITER, RT, U;
  int epi;
  QXOut oq;            // re-quantization of the output (single-matrix launches)
  const float *oq_norm;
  uint64_t *arg_part;  // argmax key per epilogue wavefront (single-matrix launches)
};

bool mv_supported(const Matrix &w);
// Whether segments of these two weight types can share one matvec launch.
bool mv_mixable(int a, int b);
// Number of argmax keys a single-matrix MV_STORE launch of w writes to MVOut::arg_part.
uint32_t mv_arg_entries(const Matrix &w);
MVPlan mv_plan(const Matrix &w, const uint32_t *rows, uint32_t n, bool glu, bool quantized_out, bool normed);
// y[r] (op)= mul * sum_c W[r][c] x[c] (+ bias[r]) for each target; epilogue `epi`
// (store, residual add, or act(W x) * (W1 x) for a gated pair). `out` re-quantizes the
// result of a single-target launch.
hipError_t mv(hipStream_t s, const MVTarget *t, uint32_t n, const QXView &x, int epi, const MVOut *out = nullptr);
// Measures the launch shapes of one launch signature on `nsets` target sets of n segments
// each (sets[k * n .. k * n + n), e.g. one per layer) and keeps the fastest for later mv()
// calls with that signature. Every candidate computes the same bits. The launches write
// their outputs as mv() would (residual adds repeat), so call it before the buffers hold
// state. Signatures already measured, F16 matrices and argmax-key launches are left alone.
hipError_t mv_tune(hipStream_t s, const MVTarget *sets, uint32_t nsets, uint32_t n, const QXView &x, int epi,
                   const MVOut *out = nullptr);
// Runs one single-matrix store launch per launch shape mv_tune may choose for it (the cost
// model's first), shape k writing y + k * rows; *count = shapes run (at most max_shapes).
hipError_t mv_shapes(hipStream_t s, const Matrix &w, const QXView &x, float *y, uint32_t max_shapes, uint32_t *count);
inline hipError_t mv(hipStream_t s, const Matrix &w, const Matrix *w1, const QXView &x, float *y, int epi,
                     const MVOut *out = nullptr) {
  MVTarget t; t.w = &w; t.w1 = w1; t.y = y;
  return mv(s, &t, 1, x, epi, out);
}

}  // namespace wgd
