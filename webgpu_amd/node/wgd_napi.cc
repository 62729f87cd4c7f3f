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
#include <string>
#include <vector>

#include "wgd.h"

namespace {

struct Ctx { wgd_context *ctx = nullptr; };
struct Model { wgd_model *m = nullptr; Ctx *owner = nullptr; int32_t vocab = 0; };

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
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok) return nullptr;
  return (T *)p;
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
  Ctx *c = new Ctx{ctx};
  return make_external(env, c, [](napi_env, void *p, void *) { delete (Ctx *)p; });
}

// destroy(context): frees every device allocation of the context (gpu.ts:66)
napi_value destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  Ctx *c = unwrap<Ctx>(env, argv[0]);
  if (c && c->ctx) { wgd_destroy(c->ctx); c->ctx = nullptr; }
  return undefined(env);
}

Ctx *live_ctx(napi_env env, napi_value v) {
  Ctx *c = unwrap<Ctx>(env, v);
  if (!c || !c->ctx) { throw_msg(env, "WGD_E_STATE", "The GPU context was disposed."); return nullptr; }
  return c;
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
  void *caps = nullptr;
  size_t n = 0;
  if (!typed(env, argv[2], napi_int32_array, &caps, &n) || (int32_t)n != cfg.layers)
    return throw_msg(env, "WGD_E_INVALID", "capacities must be an Int32Array with one entry per layer");
  wgd_model *m = nullptr;
  CHECK(c->ctx, wgd_model_create(c->ctx, &cfg, (const int32_t *)caps, &m));
  Model *w = new Model{m, c, cfg.vocab};
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

napi_value init(napi_env env, napi_value exports) {
  const struct { const char *name; napi_callback cb; } fns[] = {
      {"create", create}, {"destroy", destroy}, {"adapterName", adapter_name}, {"memory", memory},
      {"done", done}, {"modelCreate", model_create}, {"modelTensor", model_tensor},
      {"modelReady", model_ready}, {"modelForward", model_forward}, {"modelDecode", model_decode},
      {"modelSampling", model_sampling}, {"modelDestroy", model_destroy}};
  for (auto &f : fns) {
    napi_value fn;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn);
    napi_set_named_property(env, exports, f.name, fn);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
