/* oracle_san.c — drives every entry point of the float64 oracle (oracle/oracle.c) in a
 * build with AddressSanitizer and UndefinedBehaviorSanitizer (tests/native/Makefile), so
 * that an out-of-bounds access, leak, overflow or misaligned load in the checker fails the
 * CPU suite (tests/test_sanitizers.py).
 *
 *   oracle_san ops                      the kernels on random blocks of every GGUF type,
 *                                       each against an independent statement of its result
 *   oracle_san model <bundle> <out>     prompt in chunks + greedy steps of a bundled model;
 *                                       writes f64 logits after the prompt, the tokens and
 *                                       the f64 logits of the last step
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/oracle.h"
#include "bundle.h"

static int failures = 0;
#define CHECK(cond, ...)                                       \
  do {                                                         \
    if (!(cond)) {                                             \
      fprintf(stderr, "oracle_san: %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);                            \
      fputc('\n', stderr);                                     \
      failures++;                                              \
    }                                                          \
  } while (0)

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static uint64_t rnd(void) {  /* splitmix64 */
  uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static double unif(void) { return (double)(rnd() >> 11) / 9007199254740992.0; }
/* A finite half: any sign, exponent 1..29, any mantissa. */
static uint16_t finite_half(void) {
  return (uint16_t)((rnd() & 0x8000) | ((1 + rnd() % 29) << 10) | (rnd() & 1023));
}
static void put_half(uint8_t *p, uint16_t h) { p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); }

/* Random blocks of `type` whose f16 fields are finite, so decoded values compare exactly. */
static uint8_t *random_blocks(int32_t type, int64_t count) {
  int bs = orc_block_size(type), bb = orc_block_bytes(type);
  int64_t blocks = count / bs, bytes = blocks * bb;
  uint8_t *b = (uint8_t *)malloc((size_t)bytes);
  for (int64_t i = 0; i < bytes; i++) b[i] = (uint8_t)rnd();
  for (int64_t k = 0; k < blocks; k++) {
    uint8_t *p = b + k * bb;
    if (type == 0) { float f = (float)(unif() * 2 - 1); memcpy(p, &f, 4); }
    if (type == 1) put_half(p, finite_half());
    if (type == 2 || type == 8 || type == 12 || type == 13) put_half(p, finite_half());
    if (type == 12 || type == 13) put_half(p + 2, finite_half());
    if (type == 14) put_half(p + 208, finite_half());
  }
  return b;
}

static int same(double a, double b) { return a == b || (isnan(a) && isnan(b)); }

static void check_decode(void) {
  CHECK(orc_half(0x3c00) == 1.0 && orc_half(0xc000) == -2.0, "half 1, -2");
  CHECK(orc_half(0x0001) == ldexp(1.0, -24) && orc_half(0x8000) == 0.0, "half subnormal, -0");
  CHECK(isinf(orc_half(0x7c00)) && orc_half(0xfc00) < 0 && isnan(orc_half(0x7e00)), "half inf, nan");
  CHECK(orc_half(0x7bff) == 65504.0, "half max");
  const int32_t types[] = {0, 1, 2, 8, 12, 13, 14};
  for (size_t ti = 0; ti < sizeof(types) / sizeof(types[0]); ti++) {
    int32_t type = types[ti];
    int64_t count = 3 * 256;
    uint8_t *b = random_blocks(type, count);
    double *row = (double *)malloc(sizeof(double) * count);
    float *f32 = (float *)malloc(sizeof(float) * count);
    CHECK(orc_dequant_row(b, type, count, row) == 0, "dequant_row type %d", type);
    CHECK(orc_dequant_f32(b, type, count, f32) == 0, "dequant_f32 type %d", type);
    int bad = 0;
    for (int64_t i = 0; i < count; i++) {
      double d = orc_decode(b, type, i);
      if (!same(row[i], d) || !same((double)f32[i], (double)(float)d)) bad++;
    }
    CHECK(!bad, "type %d: %d elements of the block decode differ from the element decode", type, bad);
    if (orc_block_size(type) > 1)
      CHECK(orc_dequant_row(b, type, count - 1, row) == 1, "type %d: ragged count accepted", type);
    free(b); free(row); free(f32);
  }
  double x;
  CHECK(orc_dequant_row((const uint8_t *)"", 99, 1, &x) == 1 && orc_block_size(99) == 0, "unknown type accepted");
  CHECK(isnan(orc_decode((const uint8_t *)"", 99, 0)), "unknown type decodes");
}

static void check_matmul(void) {
  const int32_t types[] = {0, 8, 12, 14};
  for (size_t ti = 0; ti < sizeof(types) / sizeof(types[0]); ti++) {
    int32_t type = types[ti];
    const int64_t cols = 512, rows = 7, batch = 3, stride = 20, base = 5, off = 1;
    uint8_t *w = random_blocks(type, cols * rows);
    float *xin = (float *)malloc(sizeof(float) * cols * (batch + off));
    for (int64_t i = 0; i < cols * (batch + off); i++) xin[i] = (float)(unif() * 2 - 1);
    double *y = (double *)malloc(sizeof(double) * stride * batch), *row = (double *)malloc(sizeof(double) * cols);
    for (int64_t i = 0; i < stride * batch; i++) y[i] = -12345.0;
    CHECK(orc_matmul(type, w, xin, y, cols, rows, stride, base, off, batch) == 0, "matmul type %d", type);
    int64_t rb = cols / orc_block_size(type) * orc_block_bytes(type);
    int bad = 0;
    for (int64_t r = 0; r < rows; r++) {
      orc_dequant_row(w + r * rb, type, cols, row);
      for (int64_t bi = 0; bi < batch; bi++) {
        double s = 0;
        for (int64_t c = 0; c < cols; c++) s += row[c] * (double)xin[(bi + off) * cols + c];
        if (y[bi * stride + base + r] != s) bad++;
      }
    }
    for (int64_t bi = 0; bi < batch; bi++)
      for (int64_t i = 0; i < stride; i++)
        if ((i < base || i >= base + rows) && y[bi * stride + i] != -12345.0) bad++;
    CHECK(!bad, "matmul type %d: %d outputs differ or stray writes", type, bad);
    CHECK(orc_matmul(type == 0 ? 8 : type, w, xin, y, 31, rows, stride, base, off, batch) == 1, "ragged cols accepted");
    free(w); free(xin); free(y); free(row);
  }
}

static void check_norm_rope(void) {
  const int64_t n = 96;
  double xv[96], wv[96], yv[96];
  for (int i = 0; i < n; i++) { xv[i] = unif() * 2 - 1; wv[i] = 0.5 + unif(); }
  orc_norm(xv, wv, yv, n, 1e-6);
  double ss = 0, zz = 0;
  for (int i = 0; i < n; i++) { ss += xv[i] * xv[i]; zz += (yv[i] / wv[i]) * (yv[i] / wv[i]); }
  CHECK(fabs(zz / n - ss / (ss + n * 1e-6)) < 1e-12, "norm: mean square of y/w is %.17g", zz / n);

  const int64_t heads = 3, hd = 16, batch = 2;
  for (int mode = 0; mode < 3; mode++)
    for (int64_t rot = 8; rot <= hd; rot += 8) {
      double v[3 * 16 * 2], orig[3 * 16 * 2], ones[16];
      for (int i = 0; i < 16; i++) ones[i] = 1.0;
      for (int i = 0; i < heads * hd * batch; i++) v[i] = orig[i] = unif() * 2 - 1;
      orc_rope(v, mode == 0 ? ones : NULL, heads, hd, 4, 10000.0, 1.0, 1e-6, rot == hd ? 0 : rot, batch, mode);
      for (int64_t t = 0; t < batch * heads; t++) {
        const double *a = orig + t * hd, *b = v + t * hd;
        double inv = 1.0;
        if (mode == 0) {
          double s = 0; for (int i = 0; i < hd; i++) s += a[i] * a[i];
          inv = 1.0 / sqrt(s / hd + 1e-6);
        }
        for (int64_t i = 0; i < rot / 2; i++) {  /* rotation keeps each pair's length */
          int64_t p = mode == 2 ? 2 * i : i, q = mode == 2 ? 2 * i + 1 : i + rot / 2;
          double before = (a[p] * a[p] + a[q] * a[q]) * inv * inv, after = b[p] * b[p] + b[q] * b[q];
          CHECK(fabs(before - after) < 1e-12, "rope mode %d rot %lld: pair length changed", mode, (long long)rot);
        }
        for (int64_t i = rot; i < hd; i++)  /* the tail is only normalised */
          CHECK(fabs(b[i] - a[i] * inv) < 1e-15, "rope mode %d: tail changed", mode);
      }
    }
  double z[16], z0[16];
  for (int i = 0; i < 16; i++) z[i] = z0[i] = unif();
  orc_rope(z, NULL, 1, 16, 0, 10000.0, 1.0, 0, 0, 1, 1);  /* position 0: angle 0 */
  CHECK(!memcmp(z, z0, sizeof(z)), "rope at position 0 moved the vector");
}

static void check_attention(void) {
  const int64_t heads = 4, kvh = 2, hd = 8, cap = 5, start = 7, batch = 3, kvs = kvh * hd;
  double q[3 * 4 * 8], k[5 * 2 * 8], v[5 * 2 * 8], y[3 * 4 * 8];
  for (int i = 0; i < batch * heads * hd; i++) q[i] = unif() * 2 - 1;
  for (int i = 0; i < cap * kvs; i++) { k[i] = unif() * 2 - 1; v[i] = unif() * 2 - 1; }
  /* window 1: each query sees only its own position, slot (start + b) % cap */
  orc_attention(q, k, v, y, heads, kvh, hd, start, 0.35, 1, cap, batch);
  for (int64_t b = 0; b < batch; b++)
    for (int64_t h = 0; h < heads; h++)
      CHECK(!memcmp(y + (b * heads + h) * hd, v + ((start + b) % cap) * kvs + (h / 2) * hd, hd * sizeof(double)),
            "attention window 1: token %lld head %lld is not its own value row", (long long)b, (long long)h);
  /* a full ring: outputs are convex combinations of the value rows of the group's kv head */
  orc_attention(q, k, v, y, heads, kvh, hd, start, 0.35, cap, cap, batch);
  for (int64_t b = 0; b < batch; b++)
    for (int64_t h = 0; h < heads; h++)
      for (int64_t d = 0; d < hd; d++) {
        double lo = 1e9, hi = -1e9;
        for (int64_t t = 0; t < cap; t++) {
          double e = v[t * kvs + (h / 2) * hd + d];
          lo = e < lo ? e : lo; hi = e > hi ? e : hi;
        }
        double o = y[(b * heads + h) * hd + d];
        CHECK(o >= lo - 1e-15 && o <= hi + 1e-15, "attention output outside the value hull");
      }
  /* equal keys: softmax is uniform, output = mean of the window's values */
  double k1[5 * 2 * 8];
  for (int i = 0; i < cap * kvs; i++) k1[i] = 0.25;
  orc_attention(q, k1, v, y, heads, kvh, hd, 2, 1.0, 100, cap, 1);  /* keys 0..2 */
  for (int64_t h = 0; h < heads; h++)
    for (int64_t d = 0; d < hd; d++) {
      double m = 0; for (int t = 0; t < 3; t++) m += v[t * kvs + (h / 2) * hd + d];
      CHECK(fabs(y[h * hd + d] - m / 3) < 1e-15, "uniform attention is not the mean");
    }
}

static void check_argmax(void) {
  float l[] = {NAN, 1.f, 3.f, 3.f, INFINITY, -INFINITY, 2.f};
  CHECK(orc_argmax(l, 7) == 2, "argmax picks %lld", (long long)orc_argmax(l, 7));
  float nans[] = {NAN, INFINITY, -INFINITY};
  CHECK(orc_argmax(nans, 3) == -1 && orc_argmax(nans, 0) == -1, "argmax of no finite value");
}

static int64_t argmax_d(const double *x, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; i++) if (x[i] > x[best]) best = i;
  return best;
}

static int run_model(const char *path, const char *out) {
  bundle b;
  if (bundle_read(path, &b)) { fprintf(stderr, "oracle_san: cannot read bundle %s\n", path); return 2; }
  if (b.orc_cfg_size != sizeof(orc_config)) { fprintf(stderr, "oracle_san: config size mismatch\n"); bundle_free(&b); return 2; }
  orc_config cfg;
  memcpy(&cfg, b.orc_cfg, sizeof cfg);
  orc_model *m = orc_model_create(&cfg, b.capacities);
  for (uint32_t i = 0; i < b.n_tensors; i++) {
    const bundle_tensor *t = &b.tensors[i];
    orc_model_tensor(m, t->name, t->type, (int64_t)t->dims[0], t->n_dims > 1 ? (int64_t)t->dims[1] : 1, t->data);
  }
  int rc = 0;
  double *logits = (double *)malloc(sizeof(double) * cfg.vocab);
  int32_t *tokens = (int32_t *)calloc(b.steps + 1, sizeof(int32_t));
  int32_t bad_id[2] = {0, cfg.vocab};
  CHECK(orc_model_forward(m, bad_id, 2, 0, logits) == 1, "forward accepted an id past the vocabulary");
  for (uint32_t i = 0; i < b.n_prompt && !rc; i += b.chunk) {
    int32_t n = (int32_t)(b.n_prompt - i < b.chunk ? b.n_prompt - i : b.chunk);
    rc = orc_model_forward(m, b.prompt + i, n, (int32_t)i, i + n == b.n_prompt ? logits : NULL);
  }
  if (!rc) rc = bundle_write(out, logits, sizeof(double) * cfg.vocab, "wb");
  int32_t pos = (int32_t)b.n_prompt;
  for (uint32_t s = 0; s < b.steps && !rc; s++) {
    tokens[s] = (int32_t)argmax_d(logits, cfg.vocab);
    if (s + 1 < b.steps) rc = orc_model_forward(m, &tokens[s], 1, pos++, logits);
  }
  if (!rc) rc = bundle_write(out, tokens, sizeof(int32_t) * b.steps, "ab");
  if (!rc) rc = bundle_write(out, logits, sizeof(double) * cfg.vocab, "ab");
  CHECK(rc == 0, "model run failed (%d)", rc);
  free(logits); free(tokens);
  orc_model_destroy(m);
  bundle_free(&b);
  return 0;
}

int main(int argc, char **argv) {
  if (argc == 2 && !strcmp(argv[1], "ops")) {
    check_decode(); check_matmul(); check_norm_rope(); check_attention(); check_argmax();
  } else if (argc == 4 && !strcmp(argv[1], "model")) {
    int rc = run_model(argv[2], argv[3]);
    if (rc) return rc;
  } else {
    fprintf(stderr, "usage: oracle_san ops | model <bundle> <out>\n");
    return 2;
  }
  if (failures) { fprintf(stderr, "oracle_san: %d checks failed\n", failures); return 1; }
  printf("oracle_san %s: ok\n", argv[1]);
  return 0;
}
