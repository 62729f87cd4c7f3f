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
// 16-row tiles. Layout in one buffer of qx_bytes(K), Kp = K rounded up to 64:
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

// x (length K, K % 16 == 0) -> QX; with norm_w the stored values are x * norm_w.
hipError_t quantize(hipStream_t s, const float *x, uint32_t K, const float *norm_w, const QXOut &q);

enum MVEpilogue : int { MV_STORE = 0, MV_ADD = 1, MV_SILU = 2, MV_GELU = 3 };

// Re-quantization of a matvec's output for the next consumer: the stored vector is
// y * norm_w when norm_w is set (the consumer then applies the RMSNorm multiplier).
struct MVOut {
  QXOut q;
  const float *norm_w = nullptr;
};

// One matrix of a launch. Several matrices of one type that read the same activation
// (the Q and K projections) run in one launch, one row-tile range each.
struct MVTarget {
  const Matrix *w = nullptr;
  const Matrix *w1 = nullptr;  // the up matrix of a gated pair (MV_SILU / MV_GELU)
  float *y = nullptr;
  const float *bias = nullptr;
};

// Launch shape: a workgroup owns RT rows; its NS x NR wavefronts split K into NS slices and
// the rows into NR groups. Wc lanes share a row (P = 64 / Wc rows per load instruction);
// each lane owns NSB chunk columns of its slice and walks ITER row steps of its group, D
// row steps in flight.
struct MVPlan { uint32_t C, Wc, P, NS, NSB, NR, ITER, D, RT, tiles, threads; };

constexpr int MV_MAX_SEGS = 3;
struct MVSeg {
  const uint8_t *w, *w1;
  uint32_t bytes;      // allocation size (buffer range)
  uint32_t nbt;        // blocks in the matrix (plane offsets)
  float *y;
  const float *bias;
  uint32_t rows, tiles;
};
struct MV {
  MVSeg seg[MV_MAX_SEGS];
  uint32_t nseg;
  QXView x;
  uint32_t C, Wc, wshift, P, NS, NR, ITER, RT;
  int epi;
  QXOut oq;               // re-quantization of the output (single-matrix launches)
  const float *oq_norm;
};

bool mv_supported(const Matrix &w);
MVPlan mv_plan(const Matrix &w, const uint32_t *rows, uint32_t n, bool glu, bool quantized_out);
// y[r] (op)= mul * sum_c W[r][c] x[c] (+ bias[r]) for each target; epilogue `epi`
// (store, residual add, or act(W x) * (W1 x) for a gated pair). `out` re-quantizes the
// result of a single-target launch.
hipError_t mv(hipStream_t s, const MVTarget *t, uint32_t n, const QXView &x, int epi, const MVOut *out = nullptr);
inline hipError_t mv(hipStream_t s, const Matrix &w, const Matrix *w1, const QXView &x, float *y, int epi,
                     const MVOut *out = nullptr) {
  MVTarget t; t.w = &w; t.w1 = w1; t.y = y;
  return mv(s, &t, 1, x, epi, out);
}

}  // namespace wgd
