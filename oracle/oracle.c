/*
 * oracle.c — float64 CPU restatement of the reference's dense-decoder path.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for every parity test and the
 * timed CPU baseline. The product never links or calls it.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ quant.ts */

/* halfToFloat, src/core/quant.ts:2-5. */
double orc_half(uint16_t h) {
  double sign = (h & 0x8000) ? -1.0 : 1.0;
  int exponent = (h >> 10) & 31, fraction = h & 1023;
  if (exponent == 0) return sign * ldexp(1.0, -14) * fraction / 1024.0;
  if (exponent == 31) return fraction ? NAN : sign * INFINITY;
  return sign * ldexp(1.0, exponent - 15) * (1.0 + fraction / 1024.0);
}

/* Round to binary16: 11 significant bits for |x| >= 2^-14, a fixed 2^-24 step below
 * (subnormals); nearbyint rounds ties to even in the default rounding mode. Values at or
 * past 65520 (half an ulp above the largest half, 65504) overflow to infinity. */
double orc_round_f16(double x) {
  if (x == 0 || isnan(x) || isinf(x)) return x;
  const double a = fabs(x);
  if (a >= 65520.0) return x > 0 ? INFINITY : -INFINITY;
  int e;
  frexp(a, &e);                                  /* a = m * 2^e, 0.5 <= m < 1 */
  const double ulp = e - 1 >= -14 ? ldexp(1.0, e - 11) : ldexp(1.0, -24);
  return copysign(nearbyint(a / ulp) * ulp, x);
}

static double f16at(const uint8_t *b, int64_t p) { return orc_half((uint16_t)(b[p] | (b[p + 1] << 8))); }

/* decodeWeight, src/core/quant.ts:6-29: one element, literal restatement. */
double orc_decode(const uint8_t *b, int32_t type, int64_t i) {
  if (type == 0) { float f; memcpy(&f, b + i * 4, 4); return f; }
  if (type == 1) return f16at(b, i * 2);
  if (type == 2) {
    int64_t p = (i / 32) * 18, j = i % 32;
    return f16at(b, p) * (double)(((b[p + 2 + j % 16] >> (j < 16 ? 0 : 4)) & 15) - 8);
  }
  if (type == 8) {
    int64_t p = (i / 32) * 34; int q = b[p + 2 + i % 32];
    return f16at(b, p) * (double)(q > 127 ? q - 256 : q);
  }
  if (type == 12 || type == 13) {
    int64_t p = (i / 256) * (type == 12 ? 144 : 176), j = i % 256, s = j / 32;
    int sc = s < 4 ? (b[p + 4 + s] & 63) : ((b[p + 8 + s] & 15) | ((b[p + s] >> 6) << 4));
    int mn = s < 4 ? (b[p + 8 + s] & 63) : ((b[p + 8 + s] >> 4) | ((b[p + 4 + s] >> 6) << 4));
    int q = (b[p + (type == 12 ? 16 : 48) + (j / 64) * 32 + j % 32] >> ((s % 2) * 4)) & 15;
    if (type == 13) q |= ((b[p + 16 + j % 32] >> s) & 1) << 4;
    return f16at(b, p) * sc * q - f16at(b, p + 2) * mn;
  }
  if (type == 14) {
    int64_t p = (i / 256) * 210, j = i % 256, seg = j / 128, qtr = (j % 128) / 32, ln = j % 32;
    int lo = (b[p + seg * 64 + (qtr % 2) * 32 + ln] >> ((qtr / 2) * 4)) & 15;
    int hi = (b[p + 128 + seg * 32 + ln] >> (qtr * 2)) & 3;
    int sc = b[p + 192 + seg * 8 + qtr * 2 + ln / 16];
    return f16at(b, p + 208) * (double)(sc > 127 ? sc - 256 : sc) * (double)((lo | (hi << 4)) - 32);
  }
  return NAN;
}

int orc_block_size(int32_t type) {
  switch (type) { case 0: case 1: return 1; case 2: case 8: return 32; case 12: case 13: case 14: return 256; }
  return 0;
}
int orc_block_bytes(int32_t type) {
  switch (type) { case 0: return 4; case 1: return 2; case 2: return 18; case 8: return 34;
    case 12: return 144; case 13: return 176; case 14: return 210; }
  return 0;
}

/* Whole-block decode from the block layouts (the same formulas, hoisted per block so
 * that rows decode at memory speed). tests/test_oracle.py pins it against orc_decode. */
int orc_dequant_row(const uint8_t *b, int32_t type, int64_t count, double *out) {
  int bs = orc_block_size(type), bb = orc_block_bytes(type);
  if (!bs || count % bs) return 1;
  int64_t blocks = count / bs;
  if (type == 0) { for (int64_t i = 0; i < count; i++) { float f; memcpy(&f, b + 4 * i, 4); out[i] = f; } return 0; }
  if (type == 1) { for (int64_t i = 0; i < count; i++) out[i] = f16at(b, 2 * i); return 0; }
  for (int64_t k = 0; k < blocks; k++) {
    const uint8_t *p = b + k * bb; double *o = out + k * bs;
    if (type == 2) {
      double d = f16at(p, 0);
      for (int j = 0; j < 16; j++) { o[j] = d * (double)((p[2 + j] & 15) - 8); o[j + 16] = d * (double)((p[2 + j] >> 4) - 8); }
    } else if (type == 8) {
      double d = f16at(p, 0);
      for (int j = 0; j < 32; j++) o[j] = d * (double)(int8_t)p[2 + j];
    } else if (type == 12 || type == 13) {
      double d = f16at(p, 0), dm = f16at(p, 2);
      const uint8_t *qs = p + (type == 12 ? 16 : 48);
      for (int s = 0; s < 8; s++) {
        int sc, mn;
        if (s < 4) { sc = p[4 + s] & 63; mn = p[8 + s] & 63; }
        else { sc = (p[8 + s] & 15) | ((p[s] >> 6) << 4); mn = (p[8 + s] >> 4) | ((p[4 + s] >> 6) << 4); }
        double a = d * sc, m = dm * mn;
        const uint8_t *g = qs + (s / 2) * 32;
        for (int l = 0; l < 32; l++) {
          int q = (g[l] >> (4 * (s & 1))) & 15;
          if (type == 13) q |= ((p[16 + l] >> s) & 1) << 4;
          o[s * 32 + l] = a * q - m;
        }
      }
    } else if (type == 14) {
      double d = f16at(p, 208);
      for (int seg = 0; seg < 2; seg++)
        for (int qtr = 0; qtr < 4; qtr++)
          for (int l = 0; l < 32; l++) {
            int lo = (p[seg * 64 + (qtr & 1) * 32 + l] >> (4 * (qtr >> 1))) & 15;
            int hi = (p[128 + seg * 32 + l] >> (2 * qtr)) & 3;
            double sc = (double)(int8_t)p[192 + seg * 8 + qtr * 2 + l / 16];
            o[seg * 128 + qtr * 32 + l] = d * sc * (double)((lo | (hi << 4)) - 32);
          }
    } else return 1;
  }
  return 0;
}

int orc_dequant_f32(const uint8_t *b, int32_t type, int64_t count, float *out) {
  double *tmp = (double *)malloc(sizeof(double) * (size_t)count);
  if (!tmp) return 1;
  int rc = orc_dequant_row(b, type, count, tmp);
  for (int64_t i = 0; !rc && i < count; i++) out[i] = (float)tmp[i];
  free(tmp);
  return rc;
}

static int64_t row_bytes(int32_t type, int64_t cols) { return cols / orc_block_size(type) * orc_block_bytes(type); }

/* matmulShader semantics (shaders.ts:39-54) with an f64 sum. */
int orc_matmul(int32_t type, const uint8_t *w, const float *x, double *y, int64_t cols,
               int64_t rows, int64_t stride, int64_t row_base, int64_t input_offset,
               int64_t batch) {
  if (!orc_block_size(type) || cols % orc_block_size(type)) return 1;
  int64_t rb = row_bytes(type, cols);
  int bad = 0;
#pragma omp parallel
  {
    double *row = (double *)malloc(sizeof(double) * (size_t)cols);
    if (!row) bad = 1;
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
      if (!row) continue;
      orc_dequant_row(w + r * rb, type, cols, row);
      for (int64_t b = 0; b < batch; b++) {
        const float *xb = x + (b + input_offset) * cols; double s = 0;
        for (int64_t c = 0; c < cols; c++) s += row[c] * (double)xb[c];
        y[b * stride + row_base + r] = s;
      }
    }
    free(row);
  }
  return bad;
}

/* normShader / rms() of verify-dense.mjs:139-143. */
void orc_norm(const double *x, const double *w, double *y, int64_t n, double eps) {
  double s = 0; for (int64_t i = 0; i < n; i++) s += x[i] * x[i];
  double inv = 1.0 / sqrt(s / (double)n + eps);
  for (int64_t i = 0; i < n; i++) y[i] = x[i] * inv * w[i];
}

/* ropeShader (mode 0), ropeNeoxShader (1), ropeClassicShader (2): shaders.ts:69-87,
 * 139-168; angle (start+t)*scale/theta^(2i/rot), rot = rotary_dim or hd. */
void orc_rope(double *x, const double *w, int64_t heads, int64_t hd, int64_t start,
              double theta, double scale, double eps, int64_t rotary_dim, int64_t batch,
              int32_t mode) {
  int64_t rot = rotary_dim ? rotary_dim : hd;
  for (int64_t t = 0; t < batch; t++)
    for (int64_t h = 0; h < heads; h++) {
      double *v = x + (t * heads + h) * hd;
      if (mode == 0) {
        double s = 0; for (int64_t i = 0; i < hd; i++) s += v[i] * v[i];
        double inv = 1.0 / sqrt(s / (double)hd + eps);
        for (int64_t i = 0; i < hd; i++) v[i] = v[i] * w[i] * inv;
      }
      for (int64_t i = 0; i < rot / 2; i++) {
        double angle = (double)(start + t) * scale / pow(theta, (double)(2 * i) / (double)rot);
        double c = cos(angle), s = sin(angle);
        int64_t a = mode == 2 ? 2 * i : i, b = mode == 2 ? 2 * i + 1 : i + rot / 2;
        double l = v[a], r = v[b];
        v[a] = l * c - r * s; v[b] = l * s + r * c;
      }
    }
}

/* attentionShader semantics (shaders.ts:88-122) as a two-pass f64 softmax
 * (src/verify-context.ts:31-40): keys [end - min(end, window), end), slot t % capacity. */
void orc_attention(const double *q, const double *k, const double *v, double *y, int64_t heads,
                   int64_t kv_heads, int64_t hd, int64_t start, double scale, int64_t window,
                   int64_t capacity, int64_t batch) {
  int64_t group = heads / kv_heads, kvs = kv_heads * hd;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < batch; b++)
    for (int64_t h = 0; h < heads; h++) {
      int64_t end = start + b + 1, begin = end - (end < window ? end : window), kh = h / group;
      const double *qv = q + (b * heads + h) * hd;
      double *out = y + (b * heads + h) * hd;
      double *sc = (double *)malloc(sizeof(double) * (size_t)(end - begin));
      double mx = -INFINITY;
      for (int64_t t = begin; t < end; t++) {
        const double *kv = k + (t % capacity) * kvs + kh * hd; double dot = 0;
        for (int64_t d = 0; d < hd; d++) dot += qv[d] * kv[d];
        sc[t - begin] = dot * scale; if (sc[t - begin] > mx) mx = sc[t - begin];
      }
      double total = 0;
      for (int64_t t = begin; t < end; t++) { sc[t - begin] = exp(sc[t - begin] - mx); total += sc[t - begin]; }
      for (int64_t d = 0; d < hd; d++) out[d] = 0;
      for (int64_t t = begin; t < end; t++) {
        const double *vv = v + (t % capacity) * kvs + kh * hd; double p = sc[t - begin] / total;
        for (int64_t d = 0; d < hd; d++) out[d] += p * vv[d];
      }
      free(sc);
    }
}

/* sample(T=0), engine.ts:305-309: first strict maximum over finite values, -1 if none. */
int64_t orc_argmax(const float *logits, int64_t n) {
  float best = -INFINITY; int64_t id = -1;
  for (int64_t i = 0; i < n; i++) if (isfinite(logits[i]) && logits[i] > best) { best = logits[i]; id = i; }
  return id;
}

/* ------------------------------------------------------------------ model */

typedef struct { const uint8_t *data; int32_t type; int64_t ne0, ne1; } orc_tensor;
enum { T_ATTN_NORM, T_Q, T_K, T_V, T_O, T_QB, T_KB, T_VB, T_OB, T_QN, T_KN, T_POST_ATTN,
       T_FFN_NORM, T_GATE, T_UP, T_DOWN, T_POST_FFW, T_LAYER_COUNT };
static const char *LAYER_NAMES[T_LAYER_COUNT] = {
  "attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
  "attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias", "attn_q_norm.weight",
  "attn_k_norm.weight", "post_attention_norm.weight", "ffn_norm.weight", "ffn_gate.weight",
  "ffn_up.weight", "ffn_down.weight", "post_ffw_norm.weight" };

struct orc_model {
  orc_config c;
  int32_t *capacity;
  orc_tensor embd, out_norm, output;
  orc_tensor *layer; /* [layers][T_LAYER_COUNT] */
  double **kcache, **vcache;
};

orc_model *orc_model_create(const orc_config *cfg, const int32_t *capacities) {
  orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
  m->c = *cfg;
  m->capacity = (int32_t *)malloc(sizeof(int32_t) * cfg->layers);
  m->layer = (orc_tensor *)calloc((size_t)cfg->layers * T_LAYER_COUNT, sizeof(orc_tensor));
  m->kcache = (double **)calloc(cfg->layers, sizeof(double *));
  m->vcache = (double **)calloc(cfg->layers, sizeof(double *));
  for (int l = 0; l < cfg->layers; l++) {
    m->capacity[l] = capacities[l];
    size_t n = (size_t)capacities[l] * cfg->kv_heads * cfg->head_dim;
    m->kcache[l] = (double *)calloc(n, sizeof(double));
    m->vcache[l] = (double *)calloc(n, sizeof(double));
  }
  return m;
}

int orc_model_tensor(orc_model *m, const char *name, int32_t type, int64_t ne0, int64_t ne1,
                     const uint8_t *data) {
  orc_tensor t = { data, type, ne0, ne1 };
  if (!strcmp(name, "token_embd.weight")) { m->embd = t; return 0; }
  if (!strcmp(name, "output_norm.weight")) { m->out_norm = t; return 0; }
  if (!strcmp(name, "output.weight")) { m->output = t; return 0; }
  int l; char rest[128];
  if (sscanf(name, "blk.%d.%127s", &l, rest) == 2 && l >= 0 && l < m->c.layers)
    for (int k = 0; k < T_LAYER_COUNT; k++)
      if (!strcmp(rest, LAYER_NAMES[k])) { m->layer[l * T_LAYER_COUNT + k] = t; return 0; }
  return 0; /* tensors the dense path does not use are ignored, as in engine.ts */
}

void orc_model_destroy(orc_model *m) {
  if (!m) return;
  for (int l = 0; l < m->c.layers; l++) { free(m->kcache[l]); free(m->vcache[l]); }
  free(m->kcache); free(m->vcache); free(m->layer); free(m->capacity); free(m);
}

static double *vec(const orc_tensor *t, int64_t n) {
  double *v = (double *)malloc(sizeof(double) * (size_t)n);
  orc_dequant_row(t->data, t->type, n, v);
  return v;
}

/* y[b][r] = sum_c deq(W)[r][c] x[b][c] (+bias), f64, rows decoded once for all b. */
static void project(const orc_tensor *w, const double *x, double *y, int64_t n, const orc_tensor *bias) {
  int64_t cols = w->ne0, rows = w->ne1, rb = row_bytes(w->type, cols);
  double *bv = bias && bias->data ? vec(bias, rows) : NULL;
#pragma omp parallel
  {
    double *row = (double *)malloc(sizeof(double) * (size_t)cols);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
      orc_dequant_row(w->data + r * rb, w->type, cols, row);
      for (int64_t b = 0; b < n; b++) {
        const double *xb = x + b * cols; double s = 0;
        for (int64_t c = 0; c < cols; c++) s += row[c] * xb[c];
        y[b * rows + r] = s + (bv ? bv[r] : 0.0);
      }
    }
    free(row);
  }
  free(bv);
}

static void norm_rows(const double *x, const orc_tensor *w, double *y, int64_t n, int64_t dim, double eps) {
  double *wv = vec(w, dim);
  for (int64_t b = 0; b < n; b++) orc_norm(x + b * dim, wv, y + b * dim, dim, eps);
  free(wv);
}

static double silu(double g) { return g / (1.0 + exp(-g)); }
static double gelu_tanh(double g) { return 0.5 * g * (1.0 + tanh(0.7978845608 * (g + 0.044715 * g * g * g))); }

/* forward(ids, start): verify-dense.mjs:165-211 generalised (KV ring, quantized
 * weights, engine.ts:138-180/217-251 and the Gemma-3 body :158-174). */
int orc_model_forward(orc_model *m, const int32_t *ids, int32_t n, int32_t start, double *logits) {
  const orc_config *c = &m->c;
  for (int b = 0; b < n; b++)
    if (ids[b] < 0 || ids[b] >= m->embd.ne1) return 1;
  int64_t H = c->hidden, hd = c->head_dim, qd = (int64_t)c->heads * hd, kd = (int64_t)c->kv_heads * hd, F = c->intermediate;
  double *x = (double *)calloc((size_t)(n * H), sizeof(double));
  double *normed = (double *)malloc(sizeof(double) * n * H), *tmp = (double *)malloc(sizeof(double) * n * H);
  double *q = (double *)malloc(sizeof(double) * n * qd), *k = (double *)malloc(sizeof(double) * n * kd);
  double *v = (double *)malloc(sizeof(double) * n * kd), *att = (double *)malloc(sizeof(double) * n * qd);
  double *gate = (double *)malloc(sizeof(double) * n * F), *up = (double *)malloc(sizeof(double) * n * F);
  int64_t eb = row_bytes(m->embd.type, H);
  for (int b = 0; b < n; b++) {
    orc_dequant_row(m->embd.data + (int64_t)ids[b] * eb, m->embd.type, H, x + b * H);
    for (int64_t i = 0; i < H; i++) x[b * H + i] *= c->embed_scale;
  }
  for (int l = 0; l < c->layers; l++) {
    orc_tensor *T = m->layer + (size_t)l * T_LAYER_COUNT;
    int local = c->period > 1 && l % c->period != c->period - 1;
    norm_rows(x, &T[T_ATTN_NORM], normed, n, H, c->epsilon);
    project(&T[T_Q], normed, q, n, c->bias_q ? &T[T_QB] : NULL);
    project(&T[T_K], normed, k, n, c->bias_k ? &T[T_KB] : NULL);
    project(&T[T_V], normed, v, n, c->bias_v ? &T[T_VB] : NULL);
    int64_t window;
    if (c->family == 1) {
      double theta = local ? c->local_theta : c->theta, scale = local ? 1.0 : c->rope_scale;
      double *qn = vec(&T[T_QN], hd), *kn = vec(&T[T_KN], hd);
      orc_rope(q, qn, c->heads, hd, start, theta, scale, c->epsilon, 0, n, 0);
      orc_rope(k, kn, c->kv_heads, hd, start, theta, scale, c->epsilon, 0, n, 0);
      free(qn); free(kn);
      window = local ? c->window : c->context;
    } else {
      if (c->qk_norm) {
        double *qn = vec(&T[T_QN], hd), *kn = vec(&T[T_KN], hd);
        orc_rope(q, qn, c->heads, hd, start, c->theta, c->rope_scale, c->epsilon, c->rotary_dim, n, 0);
        orc_rope(k, kn, c->kv_heads, hd, start, c->theta, c->rope_scale, c->epsilon, c->rotary_dim, n, 0);
        free(qn); free(kn);
      } else {
        int mode = c->rope_adjacent ? 2 : 1;
        orc_rope(q, NULL, c->heads, hd, start, c->theta, c->rope_scale, 0, c->rotary_dim, n, mode);
        orc_rope(k, NULL, c->kv_heads, hd, start, c->theta, c->rope_scale, 0, c->rotary_dim, n, mode);
      }
      window = c->window > 0 ? c->window : c->context;
    }
    int64_t cap = m->capacity[l];
    for (int b = 0; b < n; b++) {
      int64_t slot = ((int64_t)start + b) % cap;
      memcpy(m->kcache[l] + slot * kd, k + b * kd, sizeof(double) * kd);
      memcpy(m->vcache[l] + slot * kd, v + b * kd, sizeof(double) * kd);
      if (c->kv_f16)
        for (int64_t i = 0; i < kd; i++) {
          m->kcache[l][slot * kd + i] = orc_round_f16(m->kcache[l][slot * kd + i]);
          m->vcache[l][slot * kd + i] = orc_round_f16(m->vcache[l][slot * kd + i]);
        }
    }
    orc_attention(q, m->kcache[l], m->vcache[l], att, c->heads, c->kv_heads, hd, start,
                  c->attention_scale, window, cap, n);
    project(&T[T_O], att, tmp, n, c->bias_output ? &T[T_OB] : NULL);
    if (c->family == 1) { norm_rows(tmp, &T[T_POST_ATTN], normed, n, H, c->epsilon); for (int64_t i = 0; i < n * H; i++) x[i] += normed[i]; }
    else for (int64_t i = 0; i < n * H; i++) x[i] += tmp[i];
    norm_rows(x, &T[T_FFN_NORM], normed, n, H, c->epsilon);
    project(&T[T_UP], normed, up, n, NULL);
    if (c->ffn_gate) {
      project(&T[T_GATE], normed, gate, n, NULL);
      for (int64_t i = 0; i < n * F; i++) up[i] = (c->gelu ? gelu_tanh(gate[i]) : silu(gate[i])) * up[i];
    } else {
      for (int64_t i = 0; i < n * F; i++) up[i] = silu(up[i]);
    }
    project(&T[T_DOWN], up, tmp, n, NULL);
    if (c->family == 1) { norm_rows(tmp, &T[T_POST_FFW], normed, n, H, c->epsilon); for (int64_t i = 0; i < n * H; i++) x[i] += normed[i]; }
    else for (int64_t i = 0; i < n * H; i++) x[i] += tmp[i];
  }
  if (logits) {
    norm_rows(x + (int64_t)(n - 1) * H, &m->out_norm, normed, 1, H, c->epsilon);
    project(c->tied_output || !m->output.data ? &m->embd : &m->output, normed, logits, 1, NULL);
  }
  free(x); free(normed); free(tmp); free(q); free(k); free(v); free(att); free(gate); free(up);
  return 0;
}

int orc_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
