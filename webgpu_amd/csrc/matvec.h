// matvec.h — quantized-activation format and the split-K decode matvec (matvec.hip).
#pragma once
#include "internal.h"

namespace wgd {

// A quantized activation vector of K elements ("QX"): three int8 digit planes, one f32
// scale per 32 elements, one exact f32 sum per 16 elements, and the multiplier applied to
// every dot product (1, or the RMSNorm inverse 1/sqrt(mean(y^2) + eps)). A producer that
// quantizes its output tile by tile cannot know the full-vector mean, so it leaves per-tile
// sums of squares (sq) and the consumer reduces them at its start: the kernel boundary is
// the only cross-workgroup synchronization. Layout in one buffer of qx_bytes(K):
//   d0[Kp] d1[Kp] d2[Kp] scale[Kp/32] sum16[Kp/16] QXHeader sq[QX_MAX_TILES], Kp = K up to 64.
constexpr uint32_t QX_MAX_TILES = 1024;
struct QXHeader {
  float mul;        // used when ntiles == 0
  uint32_t ntiles;  // > 0: mul = 1/sqrt(sum(sq[0..ntiles)) / len + eps)
  uint32_t len;
  float eps;
};
struct QXView {
  const int8_t *d[3];
  const float *scale, *sum16;
  const QXHeader *hdr;
  const float *sq;
};
struct QXOut {
  int8_t *d0 = nullptr, *d1 = nullptr, *d2 = nullptr;
  float *scale = nullptr, *sum16 = nullptr;
  QXHeader *hdr = nullptr;
  float *sq = nullptr;
};
uint64_t qx_bytes(uint32_t K);
QXOut qx_view(void *base, uint32_t K);
QXView qx_const(const QXOut &q);

// x (length K) -> QX, optionally as x * norm_w with mul = 1/sqrt(mean(x^2) + eps).
hipError_t quantize(hipStream_t s, const float *x, uint32_t K, const float *norm_w, float eps, const QXOut &q);

enum MVEpilogue : int { MV_STORE = 0, MV_ADD = 1, MV_SILU = 2, MV_GELU = 3 };

// Re-quantization of a matvec's output for the next consumer: the stored vector is
// y * norm_w (when norm_w is set, with mul = 1/sqrt(mean(y^2) + eps) over all rows).
struct MVOut {
  QXOut q;
  const float *norm_w = nullptr;
  float eps = 0.f;
};

struct MVPlan { uint32_t U, W, P, NS, RT, tiles_rows, R; };

struct MV {
  const uint8_t *w, *w1;
  int layout;
  uint64_t rb, nbt;
  uint32_t bpr;
  QXView x;
  uint32_t cols, rows, U, W, P, NS, RT, tiles_rows;
  float *y;
  uint32_t row_base;
  int epi;
  QXOut oq;
  const float *oq_norm;
  float oq_eps;
};

bool mv_supported(const Matrix &w);
MVPlan mv_plan(const Matrix &w, bool quantized_out);
// y[row_base + r] (op)= mul * sum_c W[r][c] x[c]; w1 != null selects the gated pair
// (epi MV_SILU / MV_GELU: y = act(W x) * (W1 x)). `out` re-quantizes the result.
hipError_t mv(hipStream_t s, const Matrix &w, const Matrix *w1, const QXView &x, float *y, uint32_t row_base,
              int epi, const MVOut *out = nullptr);

}  // namespace wgd
