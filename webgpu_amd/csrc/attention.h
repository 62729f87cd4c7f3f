// attention.h — the decode-step attention of one token (attention.hip).
#pragma once
#include "internal.h"
#include "matvec.h"

namespace wgd {

// One generated token at the device-resident position *pos: per-head Q/K RMSNorm and RoPE of
// the new q and k (rope mode as wgd::rope: 0 Q/K norm + half-split, 1 half-split, 2 adjacent
// pairs), the K/V append to ring slot pos % capacity, and attention of every query head over
// keys [pos + 1 - min(pos + 1, window), pos + 1) (attentionShader, shaders.ts:88-122):
// workgroups own (kv head, key chunk), a second launch merges the chunks. The output is
// written as f32 y[heads * hd] and, when qx.d0 is set, quantized for the O projection.
struct DecodeAttnArgs {
  const float *q, *k, *v;        // projections of the token, before RoPE: [heads][hd], [kvh][hd]
  void *kc, *vc;                 // ring [capacity][kvh][hd], f32 or (kv16) f16
  bool kv16 = false;
  const float *q_norm, *k_norm;  // mode 0 weights
  float *partial;                // decode_attention_scratch_floats()
  float *y;
  QXOut qx;
  const int32_t *pos;
  const float *rope;             // rope_table() of this position and theta
  uint32_t heads, kv_heads, hd, rot, capacity, window;
  float scale, eps;
  int mode;
};
bool decode_attention_supported(uint32_t heads, uint32_t kv_heads, uint32_t hd);
uint64_t decode_attention_scratch_floats(uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t capacity);
hipError_t decode_attention(hipStream_t s, const DecodeAttnArgs &a);
// f[i] = theta^(-2i/rot) in f64 for i < rot/2: the rotation angle of pair i at position p is
// p * scale * f[i], formed in f64 as in wgd::rope.
hipError_t rope_inv_freq(hipStream_t s, double *f, uint32_t rot, float theta);

// Rotation tables of one position for up to two thetas: table t holds cos(a_i) at [i] and
// sin(a_i) at [half + i], a_i = pos * scale_t * f_t[i] in f64, rounded to f32 once.
struct RopeTables {
  const double *freq[2];
  float *out[2];
  float scale[2];
  uint32_t half, n;
};

// The start of a decode token in one launch: the embedding row of *token (times `scale`, in
// f64) into hidden, its quantized form times norm_w (the first RMSNorm weight) into q, and
// the rotation tables of *pos.
hipError_t token_start(hipStream_t s, const Matrix &embd, const int32_t *token, const int32_t *pos, double scale,
                       float *hidden, const float *norm_w, const QXOut &q, const RopeTables &rt);

}  // namespace wgd
