// wgd_napi.cc — the N-API addon a Node host loads to drive libwgd (the reference's own
// runtime is Node: its engine calls WebGPU through src/core/gpu.ts). It is a thin layer
// over the C ABI of include/wgd.h: handles are N-API externals, typed arrays are passed
// by pointer for the duration of the call, and a non-zero status becomes a thrown Error
// carrying wgd_last_error(ctx), as Compute.check does (src/core/gpu.ts:20-27). Teardown
// is explicit (destroy / modelDestroy), like PagedEngine.dispose (engine.ts:303); the
// externals' finalizers free only the small host wrappers, never device state.
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "wgd.h"

namespace {

// The context lives in a shared record: the context handle, its models and its buffers each
// hold a reference, so a wrapper collected late never points at freed host memory, and
// destroy() (which frees the device side) leaves ctx NULL for every holder to see.
// Every wrapper starts with a tag, so a handle of one kind passed where another is expected
// is refused instead of being read as the wrong type.
struct Ctx { wgd_context *ctx = nullptr; };
using CtxRef = std::shared_ptr<Ctx>;
struct CtxHandle { static constexpr uint32_t TAG = 0x77676443; uint32_t tag = TAG; CtxRef c; };
struct Model { static constexpr uint32_t TAG = 0x7767644d; uint32_t tag = TAG; wgd_model *m = nullptr; CtxRef owner; int32_t vocab = 0; };
struct Buf { static constexpr uint32_t TAG = 0x77676442; uint32_t tag = TAG; wgd_buffer *b = nullptr; CtxRef owner; };

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value throw_msg(napi_env env, const char *code, const std::string &msg) {
  napi_throw_error(env, code, msg.c_str());
  return nullptr;
}

// Non-zero status -> Error(wgd_last_error); the code names the status class.
napi_value throw_status(napi_env env, wgd_context *ctx, int st) {
  const char *code = st == WGD_E_NONFINITE ? "WGD_E_NONFINITE" : st == WGD_E_BUDGET ? "WGD_E_BUDGET"
                     : st == WGD_E_DEVICE ? "WGD_E_DEVICE" : st == WGD_E_STATE ? "WGD_E_STATE" : "WGD_E_INVALID";
  const char *m = wgd_last_error(ctx);
  return throw_msg(env, code, m && *m ? m : "libwgd call failed");
}

#define CHECK(ctx, call)                                      \
  do {                                                        \
    int _st = (call);                                         \
    if (_st != WGD_OK) return throw_status(env, (ctx), _st);  \
  } while (0)

#define ARGS(n)                                                              \
  size_t argc = (n);                                                         \
  napi_value argv[(n) > 0 ? (n) : 1];                                        \
  napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr);                \
  if (argc < (size_t)(n)) return throw_msg(env, "WGD_E_INVALID", "missing arguments")

template <class T>
T *unwrap(napi_env env, napi_value v) {
  napi_valuetype vt;
  void *p = nullptr;
  if (napi_typeof(env, v, &vt) != napi_ok || vt != napi_external) return nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) return nullptr;
  uint32_t tag;
  std::memcpy(&tag, p, sizeof tag);
  return tag == T::TAG ? (T *)p : nullptr;
}

bool get_i32(napi_env env, napi_value v, int32_t *out) { return napi_get_value_int32(env, v, out) == napi_ok; }
bool get_f64(napi_env env, napi_value v, double *out) { return napi_get_value_double(env, v, out) == napi_ok; }

// A typed array's data pointer and element count, of the expected element type.
bool typed(napi_env env, napi_value v, napi_typedarray_type want, void **data, size_t *count) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  if (!is) return false;
  napi_typedarray_type t;
  napi_value ab;
  size_t off;
  if (napi_get_typedarray_info(env, v, &t, count, data, &ab, &off) != napi_ok) return false;
  return t == want;
}

napi_value make_external(napi_env env, void *p, void (*fin)(napi_env, void *, void *)) {
  napi_value ext;
  napi_create_external(env, p, fin, nullptr, &ext);
  return ext;
}

// create(device: number, budgetMiB: number | null) -> context
napi_value create(napi_env env, napi_callback_info info) {
  ARGS(2);
  int32_t dev = 0;
  if (!get_i32(env, argv[0], &dev)) return throw_msg(env, "WGD_E_INVALID", "device must be a number");
  napi_valuetype vt;
  napi_typeof(env, argv[1], &vt);
  uint64_t budget = 0;
  if (vt == napi_number) {
    double mib = 0;
    get_f64(env, argv[1], &mib);
    budget = (uint64_t)mib << 20;
  }
  wgd_context *ctx = nullptr;
  int st = wgd_create(dev, budget, &ctx);
  if (st != WGD_OK) return throw_status(env, ctx, st);
  CtxHandle *h = new CtxHandle();
  h->c = std::make_shared<Ctx>();
  h->c->ctx = ctx;
  return make_external(env, h, [](napi_env, void *p, void *) { delete (CtxHandle *)p; });
}

// destroy(context): frees every device allocation of the context (gpu.ts:66)
napi_value destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  CtxHandle *h = unwrap<CtxHandle>(env, argv[0]);
  if (h && h->c->ctx) { wgd_destroy(h->c->ctx); h->c->ctx = nullptr; }
  return undefined(env);
}

Ctx *live_ctx(napi_env env, napi_value v) {
  CtxHandle *h = unwrap<CtxHandle>(env, v);
  if (!h || !h->c->ctx) { throw_msg(env, "WGD_E_STATE", "The GPU context was disposed."); return nullptr; }
  return h->c.get();
}

napi_value adapter_name(napi_env env, napi_callback_info info) {
  ARGS(1);
  Ctx *c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  napi_value s;
  napi_create_string_utf8(env, wgd_adapter_name(c->ctx), NAPI_AUTO_LENGTH, &s);
  return s;
}

// memory(context) -> {allocated, peak} in bytes (the budget tracking of gpu.ts:24-30)
napi_value memory(napi_env env, napi_callback_info info) {
  ARGS(1);
  Ctx *c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  napi_value o, a, p;
  napi_create_object(env, &o);
  napi_create_double(env, (double)wgd_allocated(c->ctx), &a);
  napi_create_double(env, (double)wgd_peak(c->ctx), &p);
  napi_set_named_property(env, o, "allocated", a);
  napi_set_named_property(env, o, "peak", p);
  return o;
}

// done(context): the queue fence of Compute.done (gpu.ts:60); surfaces deferred faults
napi_value done(napi_env env, napi_callback_info info) {
  ARGS(1);
  Ctx *c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  CHECK(c->ctx, wgd_done(c->ctx));
  return undefined(env);
}

bool field_i32(napi_env env, napi_value o, const char *k, int32_t *out) {
  napi_value v;
  return napi_get_named_property(env, o, k, &v) == napi_ok && get_i32(env, v, out);
}
bool field_f64(napi_env env, napi_value o, const char *k, double *out) {
  napi_value v;
  return napi_get_named_property(env, o, k, &v) == napi_ok && get_f64(env, v, out);
}

// modelCreate(context, config, capacities: Int32Array) -> model. `config` carries the
// wgd_model_config fields by their C names.
napi_value model_create(napi_env env, napi_callback_info info) {
  ARGS(3);
  Ctx *c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  wgd_model_config cfg;
  std::memset(&cfg, 0, sizeof cfg);
  struct { const char *k; int32_t *p; } ints[] = {
      {"family", &cfg.family}, {"rope_adjacent", &cfg.rope_adjacent}, {"hidden", &cfg.hidden},
      {"intermediate", &cfg.intermediate}, {"layers", &cfg.layers}, {"heads", &cfg.heads},
      {"kv_heads", &cfg.kv_heads}, {"head_dim", &cfg.head_dim}, {"vocab", &cfg.vocab},
      {"rotary_dim", &cfg.rotary_dim}, {"window", &cfg.window}, {"period", &cfg.period},
      {"qk_norm", &cfg.qk_norm}, {"ffn_gate", &cfg.ffn_gate}, {"gelu", &cfg.gelu}, {"bias_q", &cfg.bias_q},
      {"bias_k", &cfg.bias_k}, {"bias_v", &cfg.bias_v}, {"bias_output", &cfg.bias_output},
      {"tied_output", &cfg.tied_output}, {"context", &cfg.context}, {"batch", &cfg.batch}};
  for (auto &f : ints)
    if (!field_i32(env, argv[1], f.k, f.p)) return throw_msg(env, "WGD_E_INVALID", std::string("config.") + f.k + " must be a number");
  struct { const char *k; float *p; } floats[] = {{"epsilon", &cfg.epsilon}, {"theta", &cfg.theta},
                                                  {"local_theta", &cfg.local_theta}, {"attention_scale", &cfg.attention_scale},
                                                  {"rope_scale", &cfg.rope_scale}};
  for (auto &f : floats) {
    double d;
    if (!field_f64(env, argv[1], f.k, &d)) return throw_msg(env, "WGD_E_INVALID", std::string("config.") + f.k + " must be a number");
    *f.p = (float)d;
  }
  if (!field_f64(env, argv[1], "embed_scale", &cfg.embed_scale)) return throw_msg(env, "WGD_E_INVALID", "config.embed_scale must be a number");
  // kv_f16 is optional (absent: the reference's f32 rings)
  bool has_kv = false;
  if (napi_has_named_property(env, argv[1], "kv_f16", &has_kv) == napi_ok && has_kv &&
      !field_i32(env, argv[1], "kv_f16", &cfg.kv_f16))
    return throw_msg(env, "WGD_E_INVALID", "config.kv_f16 must be a number");
  void *caps = nullptr;
  size_t n = 0;
  if (!typed(env, argv[2], napi_int32_array, &caps, &n) || (int32_t)n != cfg.layers)
    return throw_msg(env, "WGD_E_INVALID", "capacities must be an Int32Array with one entry per layer");
  wgd_model *m = nullptr;
  CHECK(c->ctx, wgd_model_create(c->ctx, &cfg, (const int32_t *)caps, &m));
  Model *w = new Model();
  w->m = m;
  w->owner = unwrap<CtxHandle>(env, argv[0])->c;
  w->vocab = cfg.vocab;
  return make_external(env, w, [](napi_env, void *p, void *) { delete (Model *)p; });
}

Model *live_model(napi_env env, napi_value v) {
  Model *w = unwrap<Model>(env, v);
  if (!w || !w->m || !w->owner || !w->owner->ctx) { throw_msg(env, "WGD_E_STATE", "Load a model first."); return nullptr; }
  return w;
}

// modelTensor(model, name, type, dims: number[], data: Uint8Array)
napi_value model_tensor(napi_env env, napi_callback_info info) {
  ARGS(5);
  Model *w = live_model(env, argv[0]);
  if (!w) return nullptr;
  size_t len = 0;
  napi_get_value_string_utf8(env, argv[1], nullptr, 0, &len);
  std::string name(len, '\0');
  napi_get_value_string_utf8(env, argv[1], &name[0], len + 1, &len);
  int32_t type = 0;
  if (!get_i32(env, argv[2], &type)) return throw_msg(env, "WGD_E_INVALID", "type must be a number");
  uint32_t nd = 0;
  napi_get_array_length(env, argv[3], &nd);
  if (nd < 1 || nd > 4) return throw_msg(env, "WGD_E_INVALID", "dims must hold 1 to 4 entries");
  uint64_t dims[4];
  for (uint32_t i = 0; i < nd; i++) {
    napi_value e;
    double d = 0;
    napi_get_element(env, argv[3], i, &e);
    if (!get_f64(env, e, &d) || d < 1) return throw_msg(env, "WGD_E_INVALID", "dims must be positive numbers");
    dims[i] = (uint64_t)d;
  }
  void *data = nullptr;
  size_t bytes = 0;
  if (!typed(env, argv[4], napi_uint8_array, &data, &bytes)) return throw_msg(env, "WGD_E_INVALID", "data must be a Uint8Array");
  CHECK(w->owner->ctx, wgd_model_tensor(w->m, name.c_str(), type, (int32_t)nd, dims, data, bytes));
  return undefined(env);
}

napi_value model_ready(napi_env env, napi_callback_info info) {
  ARGS(1);
  Model *w = live_model(env, argv[0]);
  if (!w) return nullptr;
  CHECK(w->owner->ctx, wgd_model_ready(w->m));
  return undefined(env);
}

// modelForward(model, ids: Int32Array, start, logits: Float32Array | null) -> greedy id of
// the last row (forward + sample(T=0), engine.ts:178-179, 305-309)
napi_value model_forward(napi_env env, napi_callback_info info) {
  ARGS(4);
  Model *w = live_model(env, argv[0]);
  if (!w) return nullptr;
  void *ids = nullptr;
  size_t n = 0;
  if (!typed(env, argv[1], napi_int32_array, &ids, &n) || n < 1) return throw_msg(env, "WGD_E_INVALID", "ids must be a non-empty Int32Array");
  int32_t start = 0;
  if (!get_i32(env, argv[2], &start)) return throw_msg(env, "WGD_E_INVALID", "start must be a number");
  napi_valuetype vt;
  napi_typeof(env, argv[3], &vt);
  void *logits = nullptr;
  size_t nl = 0;
  if (vt != napi_null && vt != napi_undefined && !typed(env, argv[3], napi_float32_array, &logits, &nl))
    return throw_msg(env, "WGD_E_INVALID", "logits must be a Float32Array or null");
  // the library writes vocab floats into it
  if (logits && nl < (size_t)w->vocab)
    return throw_msg(env, "WGD_E_INVALID", "logits holds " + std::to_string(nl) + " floats, the vocabulary " +
                                               std::to_string(w->vocab));
  int32_t tok = -1;
  CHECK(w->owner->ctx, wgd_model_forward(w->m, (const int32_t *)ids, (int32_t)n, start, (float *)logits, &tok));
  napi_value r;
  napi_create_int32(env, tok, &r);
  return r;
}

// modelDecode(model, token, start, count) -> Int32Array of the next `count` greedy ids
napi_value model_decode(napi_env env, napi_callback_info info) {
  ARGS(4);
  Model *w = live_model(env, argv[0]);
  if (!w) return nullptr;
  int32_t token = 0, start = 0, count = 0;
  if (!get_i32(env, argv[1], &token) || !get_i32(env, argv[2], &start) || !get_i32(env, argv[3], &count) || count < 0)
    return throw_msg(env, "WGD_E_INVALID", "token, start and count must be numbers");
  napi_value ab, arr;
  void *data = nullptr;
  napi_create_arraybuffer(env, sizeof(int32_t) * (size_t)count, &data, &ab);
  napi_create_typedarray(env, napi_int32_array, (size_t)count, ab, 0, &arr);
  CHECK(w->owner->ctx, wgd_model_decode(w->m, token, start, count, (int32_t *)data));
  return arr;
}

// modelSampling(model, temperature, topK, topP, seedHi, seedLo): the token pick of
// modelForward / modelDecode (temperature 0: greedy); the seed as two 32-bit halves
napi_value model_sampling(napi_env env, napi_callback_info info) {
  ARGS(6);
  Model *w = live_model(env, argv[0]);
  if (!w) return nullptr;
  double t = 0, p = 0, hi = 0, lo = 0;
  int32_t k = 0;
  if (!get_f64(env, argv[1], &t) || !get_i32(env, argv[2], &k) || !get_f64(env, argv[3], &p) ||
      !get_f64(env, argv[4], &hi) || !get_f64(env, argv[5], &lo) || k < 0)
    return throw_msg(env, "WGD_E_INVALID", "Invalid sampling settings.");
  const uint64_t seed = ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
  CHECK(w->owner->ctx, wgd_model_sampling(w->m, t, (uint32_t)k, p, seed));
  return undefined(env);
}

napi_value model_destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  Model *w = unwrap<Model>(env, argv[0]);
  if (w && w->m && w->owner && w->owner->ctx) wgd_model_destroy(w->m);
  if (w) w->m = nullptr;
  return undefined(env);
}

// ---------------------------------------------------------------- buffers and launchers
// One function per C-ABI entry point of include/wgd.h, arguments in the same order, the
// context first. Buffers are externals of the context that made them; sizes, offsets and
// counts are non-negative integer Numbers (exact up to 2^53).

bool get_u64(napi_env env, napi_value v, uint64_t *out) {
  double d = 0;
  if (!get_f64(env, v, &d) || !(d >= 0) || d > 9007199254740992.0 || d != (double)(uint64_t)d) return false;
  *out = (uint64_t)d;
  return true;
}
bool get_u32(napi_env env, napi_value v, uint32_t *out) {
  uint64_t u = 0;
  if (!get_u64(env, v, &u) || u > 0xFFFFFFFFull) return false;
  *out = (uint32_t)u;
  return true;
}
bool is_nullish(napi_env env, napi_value v) {
  napi_valuetype vt;
  napi_typeof(env, v, &vt);
  return vt == napi_null || vt == napi_undefined;
}

// Any typed array: its data pointer and length in bytes.
bool typed_bytes(napi_env env, napi_value v, void **data, uint64_t *bytes) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  if (!is) return false;
  napi_typedarray_type t;
  size_t count = 0, off = 0;
  napi_value ab;
  if (napi_get_typedarray_info(env, v, &t, &count, data, &ab, &off) != napi_ok) return false;
  size_t el = 1;
  switch (t) {
    case napi_int16_array: case napi_uint16_array: el = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
    default: el = 1;
  }
  *bytes = (uint64_t)count * el;
  return true;
}

// A buffer argument: a live buffer of context c (NULL allowed when `optional`). On false an
// error is pending.
bool buf_arg(napi_env env, napi_value v, const Ctx *c, wgd_buffer **out, bool optional) {
  *out = nullptr;
  if (optional && is_nullish(env, v)) return true;
  Buf *b = unwrap<Buf>(env, v);
  if (!b || !b->b || b->owner.get() != c) {
    throw_msg(env, "WGD_E_INVALID", "expected a live buffer of this context");
    return false;
  }
  *out = b->b;
  return true;
}

#define CTX_ARG() \
  Ctx *c = live_ctx(env, argv[0]); \
  if (!c) return nullptr
#define BUF_ARG(i, name) \
  wgd_buffer *name = nullptr; \
  if (!buf_arg(env, argv[i], c, &name, false)) return nullptr
#define OPT_BUF_ARG(i, name) \
  wgd_buffer *name = nullptr; \
  if (!buf_arg(env, argv[i], c, &name, true)) return nullptr
#define U32_ARG(i, name) \
  uint32_t name = 0; \
  if (!get_u32(env, argv[i], &name)) return throw_msg(env, "WGD_E_INVALID", #name " must be an integer in [0, 2^32)")
#define U64_ARG(i, name) \
  uint64_t name = 0; \
  if (!get_u64(env, argv[i], &name)) return throw_msg(env, "WGD_E_INVALID", #name " must be an integer in [0, 2^53]")
#define I32_ARG(i, name) \
  int32_t name = 0; \
  if (!get_i32(env, argv[i], &name)) return throw_msg(env, "WGD_E_INVALID", #name " must be a number")
#define F64_ARG(i, name) \
  double name = 0; \
  if (!get_f64(env, argv[i], &name)) return throw_msg(env, "WGD_E_INVALID", #name " must be a number")

napi_value wrap_buffer(napi_env env, const Ctx *c, napi_value ctx_value, wgd_buffer *b) {
  Buf *w = new Buf();
  w->b = b;
  w->owner = unwrap<CtxHandle>(env, ctx_value)->c;
  (void)c;
  return make_external(env, w, [](napi_env, void *p, void *) { delete (Buf *)p; });
}

napi_value num(napi_env env, double d) {
  napi_value r;
  napi_create_double(env, d, &r);
  return r;
}

// bufferCreate(ctx, size, label) -> buffer (Compute.buffer, gpu.ts:24-30)
napi_value buffer_create(napi_env env, napi_callback_info info) {
  ARGS(3);
  CTX_ARG();
  U64_ARG(1, size);
  std::string label = "buffer";
  if (!is_nullish(env, argv[2])) {
    size_t len = 0;
    napi_get_value_string_utf8(env, argv[2], nullptr, 0, &len);
    label.assign(len, '\0');
    napi_get_value_string_utf8(env, argv[2], &label[0], len + 1, &len);
  }
  wgd_buffer *b = nullptr;
  CHECK(c->ctx, wgd_buffer_create(c->ctx, size, label.c_str(), &b));
  return wrap_buffer(env, c, argv[0], b);
}

// bufferDestroy(ctx, buffer) (Compute.destroy, gpu.ts:31)
napi_value buffer_destroy(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG();
  Buf *w = unwrap<Buf>(env, argv[1]);
  if (!w || !w->b || w->owner.get() != c) return throw_msg(env, "WGD_E_INVALID", "expected a live buffer of this context");
  CHECK(c->ctx, wgd_buffer_destroy(c->ctx, w->b));
  w->b = nullptr;
  return undefined(env);
}

napi_value buffer_size(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG();
  BUF_ARG(1, b);
  return num(env, (double)wgd_buffer_size(b));
}

// uploadWeights(ctx, type, cols, rows, data: Uint8Array, label) -> buffer
napi_value upload_weights(napi_env env, napi_callback_info info) {
  ARGS(6);
  CTX_ARG();
  I32_ARG(1, type);
  U32_ARG(2, cols);
  U32_ARG(3, rows);
  void *data = nullptr;
  size_t bytes = 0;
  if (!typed(env, argv[4], napi_uint8_array, &data, &bytes)) return throw_msg(env, "WGD_E_INVALID", "data must be a Uint8Array");
  std::string label = "weights";
  if (!is_nullish(env, argv[5])) {
    size_t len = 0;
    napi_get_value_string_utf8(env, argv[5], nullptr, 0, &len);
    label.assign(len, '\0');
    napi_get_value_string_utf8(env, argv[5], &label[0], len + 1, &len);
  }
  wgd_buffer *b = nullptr;
  CHECK(c->ctx, wgd_upload_weights(c->ctx, type, cols, rows, data, bytes, label.c_str(), &b));
  return wrap_buffer(env, c, argv[0], b);
}

// write(ctx, buffer, offset, data: TypedArray) (Compute.write, gpu.ts:32)
napi_value write(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG();
  BUF_ARG(1, b);
  U64_ARG(2, offset);
  void *data = nullptr;
  uint64_t bytes = 0;
  if (!typed_bytes(env, argv[3], &data, &bytes)) return throw_msg(env, "WGD_E_INVALID", "data must be a typed array");
  CHECK(c->ctx, wgd_write(c->ctx, b, offset, data, bytes));
  return undefined(env);
}

// read(ctx, buffer, offset, out: TypedArray): fills `out` (Compute.read, gpu.ts:61-65)
napi_value read(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG();
  BUF_ARG(1, b);
  U64_ARG(2, offset);
  void *data = nullptr;
  uint64_t bytes = 0;
  if (!typed_bytes(env, argv[3], &data, &bytes)) return throw_msg(env, "WGD_E_INVALID", "out must be a typed array");
  CHECK(c->ctx, wgd_read(c->ctx, b, offset, data, bytes));
  return argv[3];
}

// copy(ctx, src, dst, size, srcOffset, dstOffset) (Compute.copy, gpu.ts:52-54)
napi_value copy(napi_env env, napi_callback_info info) {
  ARGS(6);
  CTX_ARG();
  BUF_ARG(1, src);
  BUF_ARG(2, dst);
  U64_ARG(3, size);
  U64_ARG(4, so);
  U64_ARG(5, dof);
  CHECK(c->ctx, wgd_copy(c->ctx, src, dst, size, so, dof));
  return undefined(env);
}

// clear(ctx, buffer) (Compute.clear, gpu.ts:55-59)
napi_value clear(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG();
  BUF_ARG(1, b);
  CHECK(c->ctx, wgd_clear(c->ctx, b));
  return undefined(env);
}

// matmul(ctx, type, w, x, y, cols, rows, stride, rowBase, inputOffset, batch)
napi_value matmul(napi_env env, napi_callback_info info) {
  ARGS(11);
  CTX_ARG();
  I32_ARG(1, type);
  BUF_ARG(2, w);
  BUF_ARG(3, x);
  BUF_ARG(4, y);
  U32_ARG(5, cols);
  U32_ARG(6, rows);
  U32_ARG(7, stride);
  U32_ARG(8, rowBase);
  U32_ARG(9, inputOffset);
  U32_ARG(10, batch);
  CHECK(c->ctx, wgd_matmul(c->ctx, type, w, x, y, cols, rows, stride, rowBase, inputOffset, batch));
  return undefined(env);
}

// quantizedBytes(cols) -> bytes of the quantized activation row
napi_value quantized_bytes(napi_env env, napi_callback_info info) {
  ARGS(1);
  U32_ARG(0, cols);
  return num(env, (double)wgd_quantized_bytes(cols));
}

// quantize(ctx, x, cols, normWeight | null, epsilon, qx)
napi_value quantize(napi_env env, napi_callback_info info) {
  ARGS(6);
  CTX_ARG();
  BUF_ARG(1, x);
  U32_ARG(2, cols);
  OPT_BUF_ARG(3, nw);
  F64_ARG(4, eps);
  BUF_ARG(5, qx);
  CHECK(c->ctx, wgd_quantize(c->ctx, x, cols, nw, (float)eps, qx));
  return undefined(env);
}

// matvec(ctx, type, w, qx, y, cols, rows, rowBase)
napi_value matvec(napi_env env, napi_callback_info info) {
  ARGS(8);
  CTX_ARG();
  I32_ARG(1, type);
  BUF_ARG(2, w);
  BUF_ARG(3, qx);
  BUF_ARG(4, y);
  U32_ARG(5, cols);
  U32_ARG(6, rows);
  U32_ARG(7, rowBase);
  CHECK(c->ctx, wgd_matvec(c->ctx, type, w, qx, y, cols, rows, rowBase));
  return undefined(env);
}

// dequant(ctx, type, w, out, count)
napi_value dequant(napi_env env, napi_callback_info info) {
  ARGS(5);
  CTX_ARG();
  I32_ARG(1, type);
  BUF_ARG(2, w);
  BUF_ARG(3, out);
  U64_ARG(4, count);
  CHECK(c->ctx, wgd_dequant(c->ctx, type, w, out, count));
  return undefined(env);
}

// norm(ctx, x, w, y, n, epsilon, batch)
napi_value norm(napi_env env, napi_callback_info info) {
  ARGS(7);
  CTX_ARG();
  BUF_ARG(1, x);
  BUF_ARG(2, w);
  BUF_ARG(3, y);
  U32_ARG(4, n);
  F64_ARG(5, eps);
  U32_ARG(6, batch);
  CHECK(c->ctx, wgd_norm(c->ctx, x, w, y, n, (float)eps, batch));
  return undefined(env);
}

// ropeNorm(ctx, x, w, heads, headDim, start, theta, scale, epsilon, rotaryDim, batch)
napi_value rope_norm(napi_env env, napi_callback_info info) {
  ARGS(11);
  CTX_ARG();
  BUF_ARG(1, x);
  BUF_ARG(2, w);
  U32_ARG(3, heads);
  U32_ARG(4, hd);
  U32_ARG(5, start);
  F64_ARG(6, theta);
  F64_ARG(7, scale);
  F64_ARG(8, eps);
  U32_ARG(9, rot);
  U32_ARG(10, batch);
  CHECK(c->ctx, wgd_rope_norm(c->ctx, x, w, heads, hd, start, (float)theta, (float)scale, (float)eps, rot, batch));
  return undefined(env);
}

// ropeNeox / ropeAdjacent(ctx, x, heads, headDim, start, theta, scale, rotaryDim, batch)
template <int ADJ>
napi_value rope_plain(napi_env env, napi_callback_info info) {
  ARGS(9);
  CTX_ARG();
  BUF_ARG(1, x);
  U32_ARG(2, heads);
  U32_ARG(3, hd);
  U32_ARG(4, start);
  F64_ARG(5, theta);
  F64_ARG(6, scale);
  U32_ARG(7, rot);
  U32_ARG(8, batch);
  if (ADJ) CHECK(c->ctx, wgd_rope_adjacent(c->ctx, x, heads, hd, start, (float)theta, (float)scale, rot, batch));
  else CHECK(c->ctx, wgd_rope_neox(c->ctx, x, heads, hd, start, (float)theta, (float)scale, rot, batch));
  return undefined(env);
}

// attention / attentionNoalloc / attentionF16kv(ctx, q, k, v, y, heads, kvHeads, headDim,
// start, scale, window, capacity, context, batch)
template <int KIND>
napi_value attention(napi_env env, napi_callback_info info) {
  ARGS(14);
  CTX_ARG();
  BUF_ARG(1, q);
  BUF_ARG(2, k);
  BUF_ARG(3, v);
  BUF_ARG(4, y);
  U32_ARG(5, heads);
  U32_ARG(6, kvHeads);
  U32_ARG(7, hd);
  U32_ARG(8, start);
  F64_ARG(9, scale);
  U32_ARG(10, window);
  U32_ARG(11, capacity);
  U32_ARG(12, context);
  U32_ARG(13, batch);
  if (KIND == 1)
    CHECK(c->ctx, wgd_attention_noalloc(c->ctx, q, k, v, y, heads, kvHeads, hd, start, (float)scale, window, capacity, context, batch));
  else if (KIND == 2)
    CHECK(c->ctx, wgd_attention_f16kv(c->ctx, q, k, v, y, heads, kvHeads, hd, start, (float)scale, window, capacity, context, batch));
  else
    CHECK(c->ctx, wgd_attention(c->ctx, q, k, v, y, heads, kvHeads, hd, start, (float)scale, window, capacity, context, batch));
  return undefined(env);
}

// kvStoreF16(ctx, src, dst, count, srcOffset, dstOffset): cacheKV's copy into an f16 ring
// (element offsets)
napi_value kv_store_f16(napi_env env, napi_callback_info info) {
  ARGS(6);
  CTX_ARG();
  BUF_ARG(1, src);
  BUF_ARG(2, dst);
  U64_ARG(3, count);
  U64_ARG(4, so);
  U64_ARG(5, dof);
  CHECK(c->ctx, wgd_kv_store_f16(c->ctx, src, dst, count, so, dof));
  return undefined(env);
}

// add(ctx, delta, state, n)
napi_value add(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG();
  BUF_ARG(1, delta);
  BUF_ARG(2, state);
  U32_ARG(3, n);
  CHECK(c->ctx, wgd_add(c->ctx, delta, state, n));
  return undefined(env);
}

// silu / gelu(ctx, gate, up, y, n)
template <int GELU>
napi_value glu(napi_env env, napi_callback_info info) {
  ARGS(5);
  CTX_ARG();
  BUF_ARG(1, g);
  BUF_ARG(2, u);
  BUF_ARG(3, y);
  U32_ARG(4, n);
  if (GELU) CHECK(c->ctx, wgd_gelu(c->ctx, g, u, y, n));
  else CHECK(c->ctx, wgd_silu(c->ctx, g, u, y, n));
  return undefined(env);
}

// biasAdd(ctx, y, b, n, width)
napi_value bias_add(napi_env env, napi_callback_info info) {
  ARGS(5);
  CTX_ARG();
  BUF_ARG(1, y);
  BUF_ARG(2, b);
  U32_ARG(3, n);
  U32_ARG(4, width);
  CHECK(c->ctx, wgd_bias_add(c->ctx, y, b, n, width));
  return undefined(env);
}

// activate(ctx, x, n)
napi_value activate(napi_env env, napi_callback_info info) {
  ARGS(3);
  CTX_ARG();
  BUF_ARG(1, x);
  U32_ARG(2, n);
  CHECK(c->ctx, wgd_activate(c->ctx, x, n));
  return undefined(env);
}

// argmax(ctx, logits, n, out | null) -> index of the first finite maximum
napi_value argmax(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG();
  BUF_ARG(1, logits);
  U32_ARG(2, n);
  OPT_BUF_ARG(3, out);
  int32_t id = -1;
  CHECK(c->ctx, wgd_argmax(c->ctx, logits, n, out, &id));
  napi_value r;
  napi_create_int32(env, id, &r);
  return r;
}

// sample(ctx, logits, n, temperature, topK, topP, seedHi, seedLo, index) -> token
napi_value sample(napi_env env, napi_callback_info info) {
  ARGS(9);
  CTX_ARG();
  BUF_ARG(1, logits);
  U32_ARG(2, n);
  F64_ARG(3, temperature);
  U32_ARG(4, topK);
  F64_ARG(5, topP);
  U32_ARG(6, seedHi);
  U32_ARG(7, seedLo);
  U32_ARG(8, index);
  int32_t tok = -1;
  CHECK(c->ctx, wgd_sample(c->ctx, logits, n, temperature, topK, topP, ((uint64_t)seedHi << 32) | seedLo, index, &tok));
  napi_value r;
  napi_create_int32(env, tok, &r);
  return r;
}

// embed(ctx, type, table, ids, out, hidden, n, scale)
napi_value embed(napi_env env, napi_callback_info info) {
  ARGS(8);
  CTX_ARG();
  I32_ARG(1, type);
  BUF_ARG(2, table);
  BUF_ARG(3, ids);
  BUF_ARG(4, out);
  U32_ARG(5, hidden);
  U32_ARG(6, n);
  F64_ARG(7, scale);
  CHECK(c->ctx, wgd_embed(c->ctx, type, table, ids, out, hidden, n, scale));
  return undefined(env);
}

napi_value init(napi_env env, napi_value exports) {
  const struct { const char *name; napi_callback cb; } fns[] = {
      {"create", create}, {"destroy", destroy}, {"adapterName", adapter_name}, {"memory", memory},
      {"done", done}, {"modelCreate", model_create}, {"modelTensor", model_tensor},
      {"modelReady", model_ready}, {"modelForward", model_forward}, {"modelDecode", model_decode},
      {"modelSampling", model_sampling}, {"modelDestroy", model_destroy},
      {"bufferCreate", buffer_create}, {"bufferDestroy", buffer_destroy}, {"bufferSize", buffer_size},
      {"uploadWeights", upload_weights}, {"write", write}, {"read", read}, {"copy", copy}, {"clear", clear},
      {"matmul", matmul}, {"quantizedBytes", quantized_bytes}, {"quantize", quantize}, {"matvec", matvec},
      {"dequant", dequant}, {"norm", norm}, {"ropeNorm", rope_norm}, {"ropeNeox", rope_plain<0>},
      {"ropeAdjacent", rope_plain<1>}, {"attention", attention<0>}, {"attentionNoalloc", attention<1>},
      {"attentionF16kv", attention<2>}, {"kvStoreF16", kv_store_f16},
      {"add", add}, {"silu", glu<0>}, {"gelu", glu<1>}, {"biasAdd", bias_add}, {"activate", activate},
      {"argmax", argmax}, {"sample", sample}, {"embed", embed}};
  for (auto &f : fns) {
    napi_value fn;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn);
    napi_set_named_property(env, exports, f.name, fn);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
