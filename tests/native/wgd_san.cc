// wgd_san.cc — drives libwgd's C ABI (include/wgd.h) from an executable whose host code, the
// library's included, is built with AddressSanitizer and UndefinedBehaviorSanitizer (device
// code is built as usual; tests/native/Makefile). Run on a GPU by tests/test_sanitizers_gpu.py:
// a heap overflow, use after free, leak or undefined operation in the host side of the
// library (argument checks, launch planning, the buffer and model bookkeeping, graph capture)
// ends the run with a report.
//
//   wgd_san api                          every entry point, with its error paths, on small
//                                        inputs; results checked against host arithmetic or
//                                        against another entry point of the same contract
//   wgd_san model <bundle> <out>         prompt in chunks, the device decode loop and one eager
//                                        step of a bundled model; writes the f32 logits after
//                                        the prompt, the tokens and the last step's logits
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "wgd.h"
#include "bundle.h"

static int failures = 0;
// stage markers go to stderr (unbuffered), so a run that is killed still shows where it was
static void stage(const char *what) { std::fprintf(stderr, "wgd_san: stage %s\n", what); }
#define CHECK(cond, ...)                                            \
  do {                                                              \
    if (!(cond)) {                                                  \
      std::fprintf(stderr, "wgd_san: %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                            \
      std::fputc('\n', stderr);                                     \
      failures++;                                                   \
    }                                                               \
  } while (0)
#define OK(call) CHECK((call) == WGD_OK, "%s failed: %s", #call, wgd_last_error(ctx))
#define FAILS(call, code) CHECK((call) == (code), "%s did not fail with %d", #call, code)

static uint64_t rng_state = 0x2545f4914f6cdd1dull;
static uint64_t rnd() {  // splitmix64
  uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static float unif() { return (float)((rnd() >> 40) * (1.0 / 16777216.0)) * 2.f - 1.f; }

static double half_to_double(uint16_t h) {
  const double sign = (h & 0x8000) ? -1.0 : 1.0;
  const int e = (h >> 10) & 31, f = h & 1023;
  if (e == 0) return sign * std::ldexp((double)f, -24);
  return sign * std::ldexp(1.0 + f / 1024.0, e - 15);  // e < 31 here: the blocks hold finite halves
}

// Q8_0 rows of `cols` (multiple of 32) with scales in [2^-10, 2^-6).
static std::vector<uint8_t> q8_0_rows(uint32_t rows, uint32_t cols) {
  std::vector<uint8_t> b((size_t)rows * cols / 32 * 34);
  for (size_t k = 0; k < b.size() / 34; k++) {
    uint8_t *p = b.data() + k * 34;
    const uint16_t h = (uint16_t)(((5 + rnd() % 4) << 10) | (rnd() & 1023));
    p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 32; j++) p[2 + j] = (uint8_t)rnd();
  }
  return b;
}
static double q8_0_at(const std::vector<uint8_t> &b, uint64_t i) {
  const uint8_t *p = b.data() + (i / 32) * 34;
  return half_to_double((uint16_t)(p[0] | (p[1] << 8))) * (double)(int8_t)p[2 + i % 32];
}

struct Buf {
  wgd_context *ctx;
  wgd_buffer *b = nullptr;
  Buf(wgd_context *c, uint64_t size, const char *label) : ctx(c) {
    if (wgd_buffer_create(c, size, label, &b) != WGD_OK) {
      std::fprintf(stderr, "wgd_san: cannot allocate %s: %s\n", label, wgd_last_error(c));
      std::exit(3);
    }
  }
  ~Buf() { if (b) wgd_buffer_destroy(ctx, b); }
  Buf(const Buf &) = delete;
  Buf &operator=(const Buf &) = delete;
  template <class T> void put(const std::vector<T> &v) { write(v.data(), v.size() * sizeof(T)); }
  void write(const void *p, uint64_t n) {
    if (wgd_write(ctx, b, 0, p, n) != WGD_OK) { std::fprintf(stderr, "wgd_san: write: %s\n", wgd_last_error(ctx)); std::exit(3); }
  }
  template <class T> std::vector<T> get(size_t n) {
    std::vector<T> v(n);
    if (wgd_read(ctx, b, 0, v.data(), n * sizeof(T)) != WGD_OK) { std::fprintf(stderr, "wgd_san: read: %s\n", wgd_last_error(ctx)); std::exit(3); }
    return v;
  }
};

static std::vector<float> randv(size_t n) {
  std::vector<float> v(n);
  for (auto &x : v) x = unif();
  return v;
}

static double max_rel(const std::vector<float> &got, const std::vector<double> &want) {
  double err = 0, mx = 0;
  for (size_t i = 0; i < want.size(); i++) { err = std::fmax(err, std::fabs(got[i] - want[i])); mx = std::fmax(mx, std::fabs(want[i])); }
  return mx > 0 ? err / mx : err;
}

static void check_context_and_buffers() {
  wgd_context *bad = nullptr;
  CHECK(wgd_create(9999, 0, &bad) != WGD_OK && !bad, "a context on device 9999");
  CHECK(std::strlen(wgd_last_error(nullptr)) > 0, "no message for the failed create");
  wgd_context *ctx = nullptr;
  CHECK(wgd_create(0, 64ull << 20, &ctx) == WGD_OK && ctx, "create with a 64 MiB budget");
  if (!ctx) return;
  CHECK(std::strlen(wgd_adapter_name(ctx)) > 0, "empty adapter name");
  const uint64_t base = wgd_allocated(ctx);
  wgd_buffer *a = nullptr, *big = nullptr;
  OK(wgd_buffer_create(ctx, 5, "five", &a));
  CHECK(a && wgd_buffer_size(a) == 8, "5 bytes round to 8, got %llu", (unsigned long long)wgd_buffer_size(a));
  FAILS(wgd_buffer_create(ctx, 65ull << 20, "too big", &big), WGD_E_BUDGET);
  CHECK(big == nullptr, "failed create left a buffer");
  const uint8_t bytes[8] = {1, 2, 3, 4, 5, 6, 7, 8};
  uint8_t back[8] = {0};
  OK(wgd_write(ctx, a, 2, bytes, 6));
  OK(wgd_read(ctx, a, 0, back, 8));
  CHECK(back[0] == 0 && back[1] == 0 && back[2] == 1 && back[7] == 6, "write at an offset");
  FAILS(wgd_write(ctx, a, 4, bytes, 5), WGD_E_INVALID);
  FAILS(wgd_write(ctx, a, UINT64_MAX - 2, bytes, 4), WGD_E_INVALID);
  FAILS(wgd_read(ctx, a, 8, back, 1), WGD_E_INVALID);
  wgd_buffer *c = nullptr;
  OK(wgd_buffer_create(ctx, 16, "copy target", &c));
  OK(wgd_copy(ctx, a, c, 8, 0, 8));
  FAILS(wgd_copy(ctx, a, c, 8, 4, 0), WGD_E_INVALID);
  FAILS(wgd_copy(ctx, a, c, 4, 0, UINT64_MAX - 1), WGD_E_INVALID);
  FAILS(wgd_copy(ctx, a, c, UINT64_MAX, 1, 0), WGD_E_INVALID);
  uint8_t back16[16] = {0};
  OK(wgd_read(ctx, c, 0, back16, 16));
  CHECK(back16[10] == 1 && back16[15] == 6 && back16[0] == 0, "copy placed bytes");
  OK(wgd_clear(ctx, c));
  OK(wgd_read(ctx, c, 0, back16, 16));
  CHECK(back16[10] == 0, "clear");
  CHECK(wgd_peak(ctx) >= wgd_allocated(ctx) && wgd_allocated(ctx) > base, "accounting");
  OK(wgd_buffer_destroy(ctx, a));
  // a handle that was destroyed is refused without being dereferenced
  FAILS(wgd_buffer_destroy(ctx, a), WGD_E_INVALID);
  FAILS(wgd_clear(ctx, a), WGD_E_INVALID);
  FAILS(wgd_copy(ctx, a, c, 4, 0, 0), WGD_E_INVALID);
  OK(wgd_buffer_destroy(ctx, c));
  CHECK(wgd_allocated(ctx) == base, "allocated after destroy %llu vs %llu", (unsigned long long)wgd_allocated(ctx),
        (unsigned long long)base);
  wgd_context *other = nullptr;
  OK(wgd_create(0, 0, &other));
  wgd_buffer *foreign = nullptr;
  if (other && wgd_buffer_create(other, 64, "foreign", &foreign) == WGD_OK) FAILS(wgd_clear(ctx, foreign), WGD_E_INVALID);
  OK(wgd_done(ctx));
  wgd_destroy(other);  // frees `foreign` with it
  wgd_destroy(ctx);
  wgd_destroy(nullptr);
}

static void check_kernels(wgd_context *ctx) {
  // ---- weights: Q8_0 decode, batch-1 matvec vs its two steps, the prompt GEMM
  const uint32_t cols = 512, rows = 48;
  std::vector<uint8_t> q = q8_0_rows(rows, cols);
  wgd_buffer *w = nullptr;
  FAILS(wgd_upload_weights(ctx, 8, cols, rows, q.data(), q.size() - 1, "short", &w), WGD_E_INVALID);
  FAILS(wgd_upload_weights(ctx, 77, cols, rows, q.data(), q.size(), "type", &w), WGD_E_INVALID);
  FAILS(wgd_upload_weights(ctx, 8, 31, rows, q.data(), q.size(), "shape", &w), WGD_E_INVALID);
  OK(wgd_upload_weights(ctx, 8, cols, rows, q.data(), q.size(), "q8_0 weights", &w));
  if (!w) return;
  Buf raw(ctx, q.size(), "raw q8_0"), deq(ctx, 4ull * cols * rows, "dequant");
  raw.put(q);
  OK(wgd_dequant(ctx, 8, raw.b, deq.b, (uint64_t)cols * rows));
  FAILS(wgd_dequant(ctx, 8, raw.b, deq.b, (uint64_t)cols * rows + 32), WGD_E_INVALID);
  {
    std::vector<float> d = deq.get<float>((size_t)cols * rows);
    int bad = 0;
    for (uint64_t i = 0; i < d.size(); i++) bad += d[i] != (float)q8_0_at(q, i);
    CHECK(!bad, "dequant: %d of %zu values differ from the block formula", bad, d.size());
  }
  const uint32_t batch = 9;
  std::vector<float> xs = randv((size_t)cols * batch);
  Buf x(ctx, 4ull * cols * batch, "x"), y(ctx, 4ull * rows * batch, "y"), y1(ctx, 4ull * rows, "y1");
  Buf qx(ctx, wgd_quantized_bytes(cols), "qx");
  x.put(xs);
  OK(wgd_matmul(ctx, 8, w, x.b, y.b, cols, rows, rows, 0, 0, batch));
  std::vector<float> yg = y.get<float>((size_t)rows * batch);
  std::vector<double> want((size_t)rows * batch);
  for (uint32_t b = 0; b < batch; b++)
    for (uint32_t r = 0; r < rows; r++) {
      double s = 0;
      for (uint32_t c = 0; c < cols; c++) s += q8_0_at(q, (uint64_t)r * cols + c) * xs[(size_t)b * cols + c];
      want[(size_t)b * rows + r] = s;
    }
  CHECK(max_rel(yg, want) < 2e-3, "prompt GEMM max-rel error %.3e", max_rel(yg, want));
  OK(wgd_matmul(ctx, 8, w, x.b, y1.b, cols, rows, rows, 0, 3, 1));
  OK(wgd_quantize(ctx, x.b, cols, nullptr, 0.f, qx.b));  // row 0 ...
  {
    Buf x3(ctx, 4ull * cols, "x row 3");
    OK(wgd_copy(ctx, x.b, x3.b, 4ull * cols, 12ull * cols, 0));
    OK(wgd_quantize(ctx, x3.b, cols, nullptr, 0.f, qx.b));  // ... replaced by row 3
  }
  Buf y2(ctx, 4ull * rows, "y2");
  OK(wgd_matvec(ctx, 8, w, qx.b, y2.b, cols, rows, 0));
  std::vector<float> a1 = y1.get<float>(rows), a2 = y2.get<float>(rows);
  CHECK(!std::memcmp(a1.data(), a2.data(), 4ull * rows), "batch-1 matmul differs from quantize + matvec");
  std::vector<double> w3(want.begin() + 3 * rows, want.begin() + 4 * rows);
  CHECK(max_rel(a1, w3) < 2e-3, "matvec max-rel error %.3e", max_rel(a1, w3));
  FAILS(wgd_matvec(ctx, 8, w, qx.b, y2.b, cols, rows, 1), WGD_E_INVALID);         // row_base + rows > y
  FAILS(wgd_matmul(ctx, 8, w, x.b, y.b, cols, rows, rows, 0, batch, 1), WGD_E_INVALID);  // input past x
  FAILS(wgd_matmul(ctx, 12, w, x.b, y.b, cols, rows, rows, 0, 0, 1), WGD_E_INVALID);     // other type
  OK(wgd_buffer_destroy(ctx, w));

  // ---- norm, rope, elementwise
  const uint32_t n = 256, nb = 3;
  std::vector<float> xv = randv(n * nb), wv = randv(n);
  Buf xb(ctx, 4 * n * nb, "xn"), wb(ctx, 4 * n, "wn"), yb(ctx, 4 * n * nb, "yn");
  xb.put(xv); wb.put(wv);
  OK(wgd_norm(ctx, xb.b, wb.b, yb.b, n, 1e-6f, nb));
  FAILS(wgd_norm(ctx, xb.b, wb.b, yb.b, n, 1e-6f, nb + 1), WGD_E_INVALID);
  {
    std::vector<float> got = yb.get<float>(n * nb);
    std::vector<double> wn(n * nb);
    for (uint32_t b = 0; b < nb; b++) {
      double s = 0;
      for (uint32_t i = 0; i < n; i++) s += (double)xv[b * n + i] * xv[b * n + i];
      const double inv = 1.0 / std::sqrt(s / n + 1e-6);
      for (uint32_t i = 0; i < n; i++) wn[b * n + i] = xv[b * n + i] * inv * wv[i];
    }
    CHECK(max_rel(got, wn) < 1e-5, "norm max-rel error %.3e", max_rel(got, wn));
  }
  const uint32_t heads = 4, hd = 64;
  std::vector<float> qv = randv(heads * hd * 2);
  Buf rb(ctx, 4 * heads * hd * 2, "rope");
  for (int mode = 0; mode < 2; mode++) {
    rb.put(qv);
    if (mode == 0) OK(wgd_rope_neox(ctx, rb.b, heads, hd, 0, 10000.f, 1.f, 0, 1));
    else OK(wgd_rope_adjacent(ctx, rb.b, heads, hd, 0, 10000.f, 1.f, 32, 1));
    std::vector<float> got = rb.get<float>(heads * hd * 2);
    CHECK(!std::memcmp(got.data(), qv.data(), 4ull * heads * hd * 2), "rope mode %d at position 0 moved values", mode);
  }
  FAILS(wgd_rope_neox(ctx, rb.b, heads, hd, 0, 10000.f, 1.f, 0, 3), WGD_E_INVALID);
  FAILS(wgd_rope_neox(ctx, rb.b, heads, hd, 0, 10000.f, 1.f, 65, 1), WGD_E_INVALID);
  {
    Buf nw(ctx, 4 * hd, "qk norm");
    std::vector<float> ones(hd, 1.f);
    nw.put(ones);
    rb.put(qv);
    OK(wgd_rope_norm(ctx, rb.b, nw.b, heads, hd, 5, 10000.f, 1.f, 1e-6f, 0, 2));
    std::vector<float> got = rb.get<float>(heads * hd * 2);
    int bad = 0;
    for (uint32_t t = 0; t < heads * 2; t++) {  // per head: unit mean square after the rotation
      double s = 0;
      for (uint32_t i = 0; i < hd; i++) s += (double)got[t * hd + i] * got[t * hd + i];
      bad += std::fabs(s / hd - 1.0) > 1e-3;
    }
    CHECK(!bad, "rope_norm: %d heads lost unit mean square", bad);
  }
  std::vector<float> gv = randv(n), uv = randv(n), bv = randv(16);
  Buf g(ctx, 4 * n, "g"), u(ctx, 4 * n, "u"), o(ctx, 4 * n, "o"), bias(ctx, 64, "bias");
  g.put(gv); u.put(uv); bias.put(bv);
  OK(wgd_silu(ctx, g.b, u.b, o.b, n));
  std::vector<float> so = o.get<float>(n);
  OK(wgd_gelu(ctx, g.b, u.b, o.b, n));
  std::vector<float> ge = o.get<float>(n);
  o.put(uv);
  OK(wgd_add(ctx, g.b, o.b, n));
  std::vector<float> ad = o.get<float>(n);
  OK(wgd_bias_add(ctx, o.b, bias.b, n, 16));
  std::vector<float> ba = o.get<float>(n);
  OK(wgd_activate(ctx, o.b, n));
  std::vector<float> ac = o.get<float>(n);
  FAILS(wgd_silu(ctx, g.b, u.b, o.b, n + 1), WGD_E_INVALID);
  FAILS(wgd_bias_add(ctx, o.b, bias.b, n, 17), WGD_E_INVALID);
  int bad = 0;
  for (uint32_t i = 0; i < n; i++) {
    const double gg = gv[i], sil = gg / (1 + std::exp(-gg)) * uv[i];
    const double gel = 0.5 * gg * (1 + std::tanh(0.7978845608 * (gg + 0.044715 * gg * gg * gg))) * uv[i];
    const double sum = (double)uv[i] + gv[i], biased = (double)ad[i] + bv[i % 16], act = ba[i] / (1 + std::exp(-(double)ba[i]));
    bad += std::fabs(so[i] - sil) > 1e-6 || std::fabs(ge[i] - gel) > 1e-6;
    bad += std::fabs(ad[i] - sum) > 1e-6 || std::fabs(ba[i] - biased) > 1e-6 || std::fabs(ac[i] - act) > 1e-6;
  }
  CHECK(!bad, "elementwise: %d values off", bad);

  // ---- attention and its allocation-free twin
  const uint32_t ah = 8, akv = 2, ahd = 64, cap = 40, start = 50, abatch = 4;
  std::vector<float> aq = randv(ah * ahd * abatch), ak = randv(cap * akv * ahd), av = randv(cap * akv * ahd);
  Buf qb(ctx, 4 * aq.size(), "q"), kb(ctx, 4 * ak.size(), "k"), vb(ctx, 4 * av.size(), "v");
  Buf o1(ctx, 4 * aq.size(), "o1"), o2(ctx, 4 * aq.size(), "o2");
  qb.put(aq); kb.put(ak); vb.put(av);
  OK(wgd_attention(ctx, qb.b, kb.b, vb.b, o1.b, ah, akv, ahd, start, 0.125f, 30, cap, 4096, abatch));
  OK(wgd_attention_noalloc(ctx, qb.b, kb.b, vb.b, o2.b, ah, akv, ahd, start, 0.125f, 30, cap, 4096, abatch));
  {
    std::vector<float> r1 = o1.get<float>(aq.size()), r2 = o2.get<float>(aq.size());
    CHECK(!std::memcmp(r1.data(), r2.data(), 4 * r1.size()), "attention_noalloc differs from attention");
    std::vector<double> wa(aq.size());
    for (uint32_t b = 0; b < abatch; b++)
      for (uint32_t h = 0; h < ah; h++) {
        const uint32_t end = start + b + 1, begin = end - 30, kh = h / (ah / akv);
        std::vector<double> sc(end - begin);
        double mx = -1e300, tot = 0;
        for (uint32_t t = begin; t < end; t++) {
          double d = 0;
          for (uint32_t i = 0; i < ahd; i++) d += (double)aq[(b * ah + h) * ahd + i] * ak[((t % cap) * akv + kh) * ahd + i];
          sc[t - begin] = d * 0.125;
          mx = std::fmax(mx, sc[t - begin]);
        }
        for (auto &s : sc) { s = std::exp(s - mx); tot += s; }
        for (uint32_t i = 0; i < ahd; i++) {
          double acc = 0;
          for (uint32_t t = begin; t < end; t++) acc += sc[t - begin] / tot * av[((t % cap) * akv + kh) * ahd + i];
          wa[(b * ah + h) * ahd + i] = acc;
        }
      }
    CHECK(max_rel(r1, wa) < 1e-5, "attention max-rel error %.3e", max_rel(r1, wa));
  }
  FAILS(wgd_attention(ctx, qb.b, kb.b, vb.b, o1.b, ah, 3, ahd, start, 0.125f, 30, cap, 4096, abatch), WGD_E_INVALID);
  FAILS(wgd_attention(ctx, qb.b, kb.b, vb.b, o1.b, ah, akv, ahd, start, 0.125f, 30, cap + 1, 4096, abatch), WGD_E_INVALID);
  FAILS(wgd_attention_noalloc(ctx, qb.b, kb.b, vb.b, o1.b, ah, akv, ahd, start, 0.125f, 30, cap, 4096, abatch + 1),
        WGD_E_INVALID);

  // ---- argmax, sampling, embedding, the read probe
  std::vector<float> logits = randv(1000);
  logits[17] = NAN; logits[400] = INFINITY; logits[700] = 5.f; logits[800] = 5.f;
  Buf lb(ctx, 4000, "logits"), ib(ctx, 4, "index");
  lb.put(logits);
  int32_t id = -2, tok = -2;
  OK(wgd_argmax(ctx, lb.b, 1000, ib.b, &id));
  CHECK(id == 700 && ib.get<int32_t>(1)[0] == 700, "argmax %d", id);
  OK(wgd_sample(ctx, lb.b, 1000, 0.0, 40, 0.9, 1, 0, &tok));
  CHECK(tok == 700, "greedy sample %d", tok);
  OK(wgd_sample(ctx, lb.b, 1000, 0.8, 40, 0.9, 1, 3, &tok));
  CHECK(tok >= 0 && tok < 1000 && std::isfinite(logits[tok]), "sampled %d", tok);
  FAILS(wgd_sample(ctx, lb.b, 1000, 2.5, 40, 0.9, 1, 3, &tok), WGD_E_INVALID);
  FAILS(wgd_sample(ctx, lb.b, 1000, 0.8, 0, 0.9, 1, 3, &tok), WGD_E_INVALID);
  std::vector<float> nans(1000, NAN);
  lb.put(nans);
  FAILS(wgd_argmax(ctx, lb.b, 1000, nullptr, &id), WGD_E_NONFINITE);
  CHECK(id == -1, "argmax over no finite value %d", id);
  std::vector<float> table = randv(64 * 10);
  std::vector<int32_t> ids = {3, 9, 0};
  Buf tb(ctx, 4 * table.size(), "table"), idb(ctx, 12, "ids"), eb(ctx, 4 * 64 * 3, "embedded");
  tb.put(table); idb.put(ids);
  OK(wgd_embed(ctx, 0, tb.b, idb.b, eb.b, 64, 3, 1.0));
  std::vector<float> e = eb.get<float>(64 * 3);
  CHECK(!std::memcmp(e.data() + 64, table.data() + 9 * 64, 256), "embed row 9");
  ids[1] = 10;
  idb.put(ids);
  FAILS(wgd_embed(ctx, 0, tb.b, idb.b, eb.b, 64, 3, 1.0), WGD_E_INVALID);
  Buf src(ctx, 1 << 20, "probe source"), pout(ctx, 4096, "probe out");
  OK(wgd_probe_read(ctx, src.b, 1 << 18, 4, 8, 64, 256, 8, pout.b, 1024));
  FAILS(wgd_probe_read(ctx, src.b, 1 << 18, 5, 8, 64, 256, 8, pout.b, 1024), WGD_E_INVALID);
  FAILS(wgd_probe_read(ctx, src.b, 1 << 18, 4, 8, 64, 256, 7, pout.b, 1024), WGD_E_INVALID);
  OK(wgd_done(ctx));
}

static int run_model(const char *path, const char *out) {
  bundle b;
  if (bundle_read(path, &b)) { std::fprintf(stderr, "wgd_san: cannot read bundle %s\n", path); return 2; }
  if (b.wgd_cfg_size != sizeof(wgd_model_config)) { std::fprintf(stderr, "wgd_san: config size mismatch\n"); bundle_free(&b); return 2; }
  wgd_model_config cfg;
  std::memcpy(&cfg, b.wgd_cfg, sizeof cfg);
  wgd_context *ctx = nullptr;
  stage("create");
  if (wgd_create(0, 0, &ctx) != WGD_OK) { std::fprintf(stderr, "wgd_san: %s\n", wgd_last_error(nullptr)); bundle_free(&b); return 3; }
  wgd_model *m = nullptr, *early = nullptr;
  OK(wgd_model_create(ctx, &cfg, b.capacities, &early));
  int32_t one = 1;
  float scratch[4];
  if (early) {  // forward before the tensors are in
    CHECK(wgd_model_forward(early, &one, 1, 0, nullptr, nullptr) == WGD_E_STATE, "forward before ready");
    FAILS(wgd_model_ready(early), WGD_E_INVALID);
    wgd_model_destroy(early);
  }
  stage("tensors");
  OK(wgd_model_create(ctx, &cfg, b.capacities, &m));
  if (!m) { wgd_destroy(ctx); bundle_free(&b); return 3; }
  for (uint32_t i = 0; i < b.n_tensors; i++) {
    const bundle_tensor *t = &b.tensors[i];
    if (std::strncmp(t->name, "blk.", 4) == 0 && std::atoi(t->name + 4) >= cfg.layers) continue;
    CHECK(wgd_model_tensor(m, t->name, t->type, (int32_t)t->n_dims, t->dims, t->data, t->bytes) == WGD_OK,
          "tensor %s: %s", t->name, wgd_last_error(ctx));
    if (i == 0) {  // a wrong byte count, a wrong shape
      FAILS(wgd_model_tensor(m, t->name, t->type, (int32_t)t->n_dims, t->dims, t->data, t->bytes - 1), WGD_E_INVALID);
      uint64_t dims[4] = {t->dims[0] * 2, t->n_dims > 1 ? t->dims[1] / 2 : 1, 1, 1};
      CHECK(wgd_model_tensor(m, t->name, t->type, (int32_t)t->n_dims, dims, t->data, t->bytes) != WGD_OK ||
                wgd_model_ready(m) != WGD_OK,
            "a reshaped token_embd was accepted");
      OK(wgd_model_tensor(m, t->name, t->type, (int32_t)t->n_dims, t->dims, t->data, t->bytes));
    }
  }
  stage("ready");
  OK(wgd_model_ready(m));
  stage("prompt");
  std::vector<float> logits(cfg.vocab);
  int32_t arg = -1;
  FAILS(wgd_model_forward(m, b.prompt, cfg.batch + 1, 0, nullptr, nullptr), WGD_E_INVALID);
  FAILS(wgd_model_forward(m, b.prompt, 2, cfg.context - 1, nullptr, nullptr), WGD_E_INVALID);
  int32_t bad_id = cfg.vocab;
  FAILS(wgd_model_forward(m, &bad_id, 1, 0, scratch, nullptr), WGD_E_INVALID);
  FAILS(wgd_model_sampling(m, 3.0, 40, 0.9, 1), WGD_E_INVALID);
  for (uint32_t i = 0; i < b.n_prompt; i += b.chunk) {
    const int32_t n = (int32_t)(b.n_prompt - i < b.chunk ? b.n_prompt - i : b.chunk);
    const bool last = i + n == b.n_prompt;
    OK(wgd_model_forward(m, b.prompt + i, n, (int32_t)i, last ? logits.data() : nullptr, last ? &arg : nullptr));
  }
  int rc = bundle_write(out, logits.data(), 4ull * cfg.vocab, "wb");
  std::vector<int32_t> tokens(b.steps > 0 ? b.steps : 1);
  tokens[0] = arg;
  const int32_t n = (int32_t)b.n_prompt, steps = (int32_t)b.steps;
  stage("decode");
  FAILS(wgd_model_decode(m, arg, n, cfg.context, tokens.data() + 1), WGD_E_INVALID);
  if (steps > 2) OK(wgd_model_decode(m, arg, n, steps - 2, tokens.data() + 1));
  if (steps > 1) OK(wgd_model_forward(m, &tokens[steps - 2], 1, n + steps - 2, logits.data(), &tokens[steps - 1]));
  if (!rc) rc = bundle_write(out, tokens.data(), 4ull * steps, "ab");
  if (!rc) rc = bundle_write(out, logits.data(), 4ull * cfg.vocab, "ab");
  CHECK(rc == 0, "writing %s", out);
  // sampled decode graph: runs, and repeats itself from the same state
  stage("sampled decode");
  OK(wgd_model_sampling(m, 0.7, 20, 0.95, 42));
  std::vector<int32_t> s1(4), s2(4);
  OK(wgd_model_decode(m, arg, n, 4, s1.data()));
  OK(wgd_model_decode(m, arg, n, 4, s2.data()));
  CHECK(s1 == s2, "sampled decode from the same state differs");
  OK(wgd_model_sampling(m, 0.0, 40, 0.9, 0));
  stage("destroy");
  wgd_model_destroy(m);
  OK(wgd_done(ctx));
  wgd_destroy(ctx);
  bundle_free(&b);
  return 0;
}

int main(int argc, char **argv) {
  std::setvbuf(stdout, nullptr, _IONBF, 0);
  if (argc == 2 && !std::strcmp(argv[1], "api")) {
    stage("contexts and buffers");
    check_context_and_buffers();
    wgd_context *ctx = nullptr;
    stage("kernels");
    if (wgd_create(0, 0, &ctx) != WGD_OK) { std::fprintf(stderr, "wgd_san: %s\n", wgd_last_error(nullptr)); return 3; }
    check_kernels(ctx);
    wgd_destroy(ctx);
  } else if (argc == 4 && !std::strcmp(argv[1], "model")) {
    const int rc = run_model(argv[2], argv[3]);
    if (rc) return rc;
  } else {
    std::fprintf(stderr, "usage: wgd_san api | model <bundle> <out>\n");
    return 2;
  }
  if (failures) { std::fprintf(stderr, "wgd_san: %d checks failed\n", failures); return 1; }
  std::printf("wgd_san %s: ok\n", argv[1]);
  stage("exit");
  return 0;
}
