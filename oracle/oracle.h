/*
 * oracle.h — CPU restatement of the reference's dense-decoder path, in float64.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the timed CPU
 * baseline; the product (libwgd.so and the webgpu_amd package) never calls it.
 *
 * What each part restates (paths relative to the reference repository):
 *   orc_half, orc_decode          src/core/quant.ts:2-29 (element-wise, literal)
 *   orc_dequant_row               block-wise decode of whole rows; pinned against
 *                                 orc_decode on every type and the quant.test.ts KATs
 *   orc_matmul                    matmulShader semantics, shaders.ts:39-54, in f64
 *   orc_norm / orc_rope_*         shaders.ts:55-87, 139-168 in f64
 *   orc_attention                 attentionShader semantics, shaders.ts:88-122, as the
 *                                 two-pass f64 softmax of src/verify-context.ts:31-40
 *   orc_model_*                   the f64 reference forward of scripts/verify-dense.mjs
 *                                 :138-211, KV-cached, with quantized weights, Q/K norm,
 *                                 biases, partial rotary, sliding windows and the Gemma-3
 *                                 body of src/core/engine.ts:158-174
 *   orc_argmax                    sample(T=0), src/core/engine.ts:305-309
 */
#ifndef WGD_ORACLE_H
#define WGD_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

double orc_half(uint16_t h);
double orc_decode(const uint8_t *data, int32_t type, int64_t i);
int orc_block_size(int32_t type);
int orc_block_bytes(int32_t type);
/* Decode `count` elements starting at element 0 of `data` (count % block == 0). */
int orc_dequant_row(const uint8_t *data, int32_t type, int64_t count, double *out);
/* Same, rounded to f32 (what the reference stores into a Float32Array). */
int orc_dequant_f32(const uint8_t *data, int32_t type, int64_t count, float *out);

int orc_matmul(int32_t type, const uint8_t *w, const float *x, double *y, int64_t cols,
               int64_t rows, int64_t stride, int64_t row_base, int64_t input_offset,
               int64_t batch);
void orc_norm(const double *x, const double *w, double *y, int64_t n, double eps);
void orc_rope(double *x, const double *w, int64_t heads, int64_t hd, int64_t start,
              double theta, double scale, double eps, int64_t rotary_dim, int64_t batch,
              int32_t mode /* 0 q/k-norm + half-split, 1 half-split, 2 adjacent */);
void orc_attention(const double *q, const double *k, const double *v, double *y, int64_t heads,
                   int64_t kv_heads, int64_t hd, int64_t start, double scale, int64_t window,
                   int64_t capacity, int64_t batch);
int64_t orc_argmax(const float *logits, int64_t n);
/* x rounded to the nearest IEEE binary16 value (ties to even; overflow to +-inf), as f64. */
double orc_round_f16(double x);

typedef struct orc_config {
  int32_t family, rope_adjacent;
  int32_t hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
  int32_t rotary_dim, window, period;
  int32_t qk_norm, ffn_gate, gelu, bias_q, bias_k, bias_v, bias_output, tied_output;
  int32_t context, batch;
  double epsilon, theta, local_theta, attention_scale, rope_scale, embed_scale;
  int32_t kv_f16; /* K/V ring values rounded to the nearest f16 (ties to even) when cached */
} orc_config;

typedef struct orc_model orc_model;
orc_model *orc_model_create(const orc_config *cfg, const int32_t *capacities);
/* Borrow a tensor's raw GGUF bytes (must outlive the model). */
int orc_model_tensor(orc_model *m, const char *name, int32_t type, int64_t ne0, int64_t ne1,
                     const uint8_t *data);
/* forward(ids, start) of n tokens; logits (vocab doubles) of the last row when non-NULL. */
int orc_model_forward(orc_model *m, const int32_t *ids, int32_t n, int32_t start,
                      double *logits);
void orc_model_destroy(orc_model *m);
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
