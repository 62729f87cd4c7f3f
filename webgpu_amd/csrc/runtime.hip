// runtime.hip — the C ABI of libwgd: the `Compute` object of src/core/gpu.ts:2-67
// (device, budget-tracked buffers, ordered writes, copies, clears, fences, read-back,
// deferred faults) and one bounds-checked launcher per WGSL pipeline of
// src/core/shaders.ts / qwen-shaders.ts. Every launcher validates that the kernel's
// accesses stay inside the buffers before anything is queued.
#include <cstdio>
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <set>
#include <string>

#include "internal.h"
#include "matvec.h"
#include "model.h"

using namespace wgd;

struct wgd_buffer {
  void *ptr = nullptr;
  uint64_t size = 0;
  std::string label;
  // Weight matrices uploaded with wgd_upload_weights remember their type, shape and layout.
  int layout = LAYOUT_GGUF, type = -1;
  uint32_t cols = 0, rows = 0;
  // Quantized activations written by wgd_quantize: length and the pending RMSNorm.
  uint32_t qx_cols = 0;
  bool qx_normed = false;
  float qx_eps = 0.f;
};

static thread_local std::string g_error;
static int scratch_setup(int device, float **out);

int wgd::fail(wgd_context *ctx, int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->error = buf; else g_error = buf;
  return code;
}

int wgd::hip_fail(wgd_context *ctx, hipError_t e, const char *what) {
  return fail(ctx, WGD_E_DEVICE, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

int wgd::ctx_alloc(wgd_context *ctx, uint64_t size, const char *label, void **out) {
  size = size < 4 ? 4 : (size + 3) / 4 * 4;
  if (ctx->allocated + size > ctx->limit)
    return fail(ctx, WGD_E_BUDGET, "GPU budget exceeded allocating %s (%llu bytes). Reduce context length or increase the memory budget.",
                label, (unsigned long long)size);
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, size);
  if (e != hipSuccess) return hip_fail(ctx, e, label);
  e = hipMemsetAsync(p, 0, size, ctx->stream);
  if (e != hipSuccess) { hipFree(p); return hip_fail(ctx, e, label); }
  ctx->allocated += size;
  if (ctx->allocated > ctx->peak) ctx->peak = ctx->allocated;
  ctx->sizes[p] = size;
  *out = p;
  return WGD_OK;
}

void wgd::ctx_free(wgd_context *ctx, void *p) {
  if (!p) return;
  auto it = ctx->sizes.find(p);
  if (it == ctx->sizes.end()) return;
  hipStreamSynchronize(ctx->stream);
  hipFree(p);
  ctx->allocated -= it->second;
  ctx->sizes.erase(it);
}

// Checks for a fault raised by earlier asynchronous work.
int wgd::ctx_check(wgd_context *ctx, hipError_t launch, const char *what) {
  if (launch != hipSuccess) return hip_fail(ctx, launch, what);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(ctx, e, what);
  return WGD_OK;
}

int wgd::ctx_sync(wgd_context *ctx, const char *what) {
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, what);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(ctx, e, what);
  return WGD_OK;
}

extern "C" {

int wgd_create(int32_t device, uint64_t budget_bytes, wgd_context **out) {
  if (!out) return fail(nullptr, WGD_E_INVALID, "wgd_create: out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(nullptr, WGD_E_DEVICE, "No HIP device is available (%s).", e == hipSuccess ? "no devices" : hipGetErrorString(e));
  if (device < 0 || device >= count) return fail(nullptr, WGD_E_INVALID, "HIP device %d does not exist (%d present).", device, count);
  e = hipSetDevice(device);
  if (e != hipSuccess) return fail(nullptr, WGD_E_DEVICE, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
  hipDeviceProp_t p;
  e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return fail(nullptr, WGD_E_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, WGD_E_DEVICE, "libwgd is built for gfx950 (MI355X); device %d is %s.", device, p.gcnArchName);
  float *static_scratch = nullptr;
  int src = scratch_setup(device, &static_scratch);
  if (src) return src;
  wgd_context *ctx = new wgd_context();
  ctx->device = device;
  ctx->noalloc_scratch = static_scratch;
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) { delete ctx; return fail(nullptr, WGD_E_DEVICE, "hipStreamCreate: %s", hipGetErrorString(e)); }
  size_t free_b = 0, total_b = 0;
  hipMemGetInfo(&free_b, &total_b);
  ctx->limit = budget_bytes ? budget_bytes : (uint64_t)free_b;
  // the marketing name can be empty (a driver that does not report it): name the device by index then
  const std::string name = p.name[0] ? std::string(p.name) : "HIP device " + std::to_string(device);
  ctx->adapter = name + " (" + p.gcnArchName + ", " + std::to_string(p.multiProcessorCount) + " CUs)";
  void *scratch = nullptr;
  if (ctx_alloc(ctx, 8 + 8 * 256, "argmax scratch", &scratch) != WGD_OK) {
    g_error = ctx->error;
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return WGD_E_BUDGET;
  }
  ctx->argmax_scratch = (int32_t *)scratch;
  *out = ctx;
  return WGD_OK;
}

void wgd_destroy(wgd_context *ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (wgd_model *m : std::set<wgd_model *>(ctx->models)) model_destroy(m);
  for (wgd_buffer *b : ctx->buffers) delete b;  // their memory is freed with ctx->sizes below
  ctx->buffers.clear();
  for (auto &kv : ctx->sizes) hipFree(kv.first);
  ctx->sizes.clear();
  hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char *wgd_last_error(const wgd_context *ctx) { return ctx ? ctx->error.c_str() : g_error.c_str(); }
const char *wgd_adapter_name(const wgd_context *ctx) { return ctx ? ctx->adapter.c_str() : ""; }
uint64_t wgd_allocated(const wgd_context *ctx) { return ctx ? ctx->allocated : 0; }
uint64_t wgd_peak(const wgd_context *ctx) { return ctx ? ctx->peak : 0; }

int wgd_buffer_create(wgd_context *ctx, uint64_t size, const char *label, wgd_buffer **out) {
  if (!ctx || !out) return fail(ctx, WGD_E_INVALID, "wgd_buffer_create: NULL argument");
  *out = nullptr;
  void *p = nullptr;
  int rc = ctx_alloc(ctx, size, label ? label : "buffer", &p);
  if (rc) return rc;
  wgd_buffer *b = new wgd_buffer();
  b->ptr = p;
  b->size = ctx->sizes[p];
  b->label = label ? label : "buffer";
  ctx->buffers.insert(b);
  *out = b;
  return WGD_OK;
}

int wgd_buffer_destroy(wgd_context *ctx, wgd_buffer *b) {
  if (!ctx || !b) return fail(ctx, WGD_E_INVALID, "wgd_buffer_destroy: NULL argument");
  if (!ctx->buffers.count(b)) return fail(ctx, WGD_E_INVALID, "wgd_buffer_destroy: buffer does not belong to this context");
  ctx_free(ctx, b->ptr);
  ctx->buffers.erase(b);
  delete b;
  return WGD_OK;
}

uint64_t wgd_buffer_size(const wgd_buffer *b) { return b ? b->size : 0; }

void *wgd_stream(const wgd_context *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int wgd_upload_weights(wgd_context *ctx, int32_t type, uint32_t cols, uint32_t rows, const void *data, uint64_t bytes,
                       const char *label, wgd_buffer **out) {
  if (!ctx || !out || !data) return fail(ctx, WGD_E_INVALID, "wgd_upload_weights: NULL argument");
  hipSetDevice(ctx->device);
  *out = nullptr;
  if (block_size(type) == 0) return fail(ctx, WGD_E_INVALID, "Unsupported tensor quantization %d.", type);
  if (!cols || !rows || cols % block_size(type)) return fail(ctx, WGD_E_INVALID, "wgd_upload_weights: invalid shape %ux%u", cols, rows);
  uint64_t need = (uint64_t)rows * row_bytes(type, cols);
  if (bytes != need) return fail(ctx, WGD_E_INVALID, "wgd_upload_weights: %llu bytes given, shape needs %llu", (unsigned long long)bytes, (unsigned long long)need);
  wgd_buffer *b = nullptr;
  int rc = wgd_buffer_create(ctx, has_planar(type, cols) ? planar_bytes(type, cols, rows) : need, label ? label : "weights", &b);
  if (rc) return rc;
  if (has_planar(type, cols)) {
    void *raw = nullptr;
    rc = ctx_alloc(ctx, need, "upload staging", &raw);
    if (!rc) rc = ctx_check(ctx, hipMemcpyAsync(raw, data, need, hipMemcpyHostToDevice, ctx->stream), "wgd_upload_weights");
    if (!rc) rc = ctx_check(ctx, repack_planar(ctx->stream, type, (const uint8_t *)raw, (uint8_t *)b->ptr, cols, rows), "wgd_upload_weights");
    if (!rc) rc = ctx_sync(ctx, "wgd_upload_weights");
    ctx_free(ctx, raw);
    b->layout = LAYOUT_PLANAR;
  } else {
    rc = ctx_check(ctx, hipMemcpyAsync(b->ptr, data, need, hipMemcpyHostToDevice, ctx->stream), "wgd_upload_weights");
    if (!rc) rc = ctx_sync(ctx, "wgd_upload_weights");
  }
  if (rc) { std::string e = ctx->error; wgd_buffer_destroy(ctx, b); ctx->error = e; return rc; }
  b->type = type; b->cols = cols; b->rows = rows;
  *out = b;
  return WGD_OK;
}

static bool owned(wgd_context *ctx, const wgd_buffer *b) { return b && ctx->buffers.count(const_cast<wgd_buffer *>(b)); }

#define NEED_CTX(ctx) do { if (!(ctx)) return fail(nullptr, WGD_E_INVALID, "NULL context"); hipSetDevice((ctx)->device); } while (0)
#define NEED_BUF(ctx, b, what) do { if (!owned(ctx, b)) return fail(ctx, WGD_E_INVALID, "%s: missing or foreign buffer", what); } while (0)
#define NEED_FIT(ctx, b, bytes, what) do { if ((uint64_t)(bytes) > (b)->size) return fail(ctx, WGD_E_INVALID, "%s: buffer %s holds %llu bytes, the launch reads or writes %llu", what, (b)->label.c_str(), (unsigned long long)(b)->size, (unsigned long long)(bytes)); } while (0)

int wgd_write(wgd_context *ctx, wgd_buffer *b, uint64_t offset, const void *data, uint64_t bytes) {
  NEED_CTX(ctx); NEED_BUF(ctx, b, "wgd_write");
  if (!bytes) return WGD_OK;
  if (!data || offset + bytes > b->size || offset + bytes < offset) return fail(ctx, WGD_E_INVALID, "wgd_write: range outside buffer %s", b->label.c_str());
  hipError_t e = hipMemcpyAsync((uint8_t *)b->ptr + offset, data, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "wgd_write");
  return ctx_sync(ctx, "wgd_write");
}

int wgd_read(wgd_context *ctx, const wgd_buffer *b, uint64_t offset, void *out, uint64_t bytes) {
  NEED_CTX(ctx); NEED_BUF(ctx, b, "wgd_read");
  if (!bytes) return ctx_sync(ctx, "wgd_read");
  if (!out || offset + bytes > b->size || offset + bytes < offset) return fail(ctx, WGD_E_INVALID, "wgd_read: range outside buffer %s", b->label.c_str());
  int rc = ctx_sync(ctx, "GPU fault before read-back");
  if (rc) return rc;
  hipError_t e = hipMemcpyAsync(out, (const uint8_t *)b->ptr + offset, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "wgd_read");
  return ctx_sync(ctx, "wgd_read");
}

int wgd_copy(wgd_context *ctx, const wgd_buffer *src, wgd_buffer *dst, uint64_t size, uint64_t so, uint64_t dof) {
  NEED_CTX(ctx); NEED_BUF(ctx, src, "wgd_copy"); NEED_BUF(ctx, dst, "wgd_copy");
  if (!size) return WGD_OK;
  if (so > src->size || size > src->size - so || dof > dst->size || size > dst->size - dof)
    return fail(ctx, WGD_E_INVALID, "wgd_copy: range outside buffers");
  return ctx_check(ctx, hipMemcpyAsync((uint8_t *)dst->ptr + dof, (const uint8_t *)src->ptr + so, size, hipMemcpyDeviceToDevice, ctx->stream), "wgd_copy");
}

int wgd_clear(wgd_context *ctx, wgd_buffer *b) {
  NEED_CTX(ctx); NEED_BUF(ctx, b, "wgd_clear");
  return ctx_check(ctx, hipMemsetAsync(b->ptr, 0, b->size, ctx->stream), "wgd_clear");
}

int wgd_done(wgd_context *ctx) {
  NEED_CTX(ctx);
  return ctx_sync(ctx, "GPU fault");
}

// ------------------------------------------------------------------ kernel launchers

static bool known_type(int t) { return block_size(t) != 0; }

int wgd_matmul(wgd_context *ctx, int32_t type, const wgd_buffer *w, const wgd_buffer *x, wgd_buffer *y,
               uint32_t cols, uint32_t rows, uint32_t stride, uint32_t row_base, uint32_t input_offset,
               uint32_t batch) {
  NEED_CTX(ctx); NEED_BUF(ctx, w, "matmul"); NEED_BUF(ctx, x, "matmul"); NEED_BUF(ctx, y, "matmul");
  if (!known_type(type)) return fail(ctx, WGD_E_INVALID, "No GPU kernel for tensor type %d.", type);
  if (!cols || cols % block_size(type)) return fail(ctx, WGD_E_INVALID, "matmul: %u columns are not a whole number of %d-element blocks", cols, block_size(type));
  if (!rows || !batch) return WGD_OK;
  NEED_FIT(ctx, w, (uint64_t)rows * row_bytes(type, cols), "matmul weights");
  NEED_FIT(ctx, x, (uint64_t)(batch + input_offset) * cols * 4, "matmul input");
  if (batch > 1 && stride < row_base + rows) return fail(ctx, WGD_E_INVALID, "matmul: stride %u < rowBase + rows", stride);
  NEED_FIT(ctx, y, ((uint64_t)(batch - 1) * stride + row_base + rows) * 4, "matmul output");
  Matrix m; m.data = (const uint8_t *)w->ptr; m.type = type; m.layout = LAYOUT_GGUF; m.cols = cols; m.rows = rows;
  if (w->layout != LAYOUT_GGUF) {
    if (w->type != type || w->cols != cols || w->rows != rows)
      return fail(ctx, WGD_E_INVALID, "matmul: weights %s were uploaded as type %d, %ux%u", w->label.c_str(), w->type, w->cols, w->rows);
    m.layout = w->layout;
  }
  if (batch == 1 && mv_supported(m)) {
    // Decode path: quantize the activation row, then the split-K integer-dot matvec.
    auto grow = [&](void **p, uint64_t *have, uint64_t need, const char *label) -> int {
      if (need <= *have) return WGD_OK;
      ctx_free(ctx, *p);
      *p = nullptr; *have = 0;
      int rc = ctx_alloc(ctx, need, label, p);  // zero-filled: the counters start at zero
      if (!rc) *have = need;
      return rc;
    };
    int rc = grow(&ctx->mv_qx, &ctx->mv_qx_bytes, qx_bytes(cols), "matvec activation");
    if (rc) return rc;
    QXOut q = qx_view(ctx->mv_qx, cols);
    rc = ctx_check(ctx, quantize(ctx->stream, (const float *)x->ptr + (uint64_t)input_offset * cols, cols, nullptr, q), "matmul");
    if (rc) return rc;
    return ctx_check(ctx, mv(ctx->stream, m, nullptr, qx_const(q, cols, false, 0.f), (float *)y->ptr + row_base, MV_STORE), "matmul");
  }
  // split-K partial sums of the prompt GEMM, grown on demand and kept with the context
  const uint64_t gp = gemm_split_floats(m, batch);
  if (gp > ctx->gemm_part_floats) {
    ctx_free(ctx, ctx->gemm_part);
    ctx->gemm_part = nullptr; ctx->gemm_part_floats = 0;
    void *p = nullptr;
    int rc = ctx_alloc(ctx, gp * 4, "GEMM split sums", &p);
    if (rc) return rc;
    ctx->gemm_part = (float *)p; ctx->gemm_part_floats = gp;
  }
  // and the bf16 split of the input, re-made on every call
  const uint64_t gx = gemm_input_elems(cols, batch);
  if (m.layout == LAYOUT_PLANAR && gx > ctx->gemm_xs_elems) {
    ctx_free(ctx, ctx->gemm_xs);
    ctx->gemm_xs = nullptr; ctx->gemm_xs_elems = 0;
    void *p = nullptr;
    int rc = ctx_alloc(ctx, gx * 2, "GEMM split input", &p);
    if (rc) return rc;
    ctx->gemm_xs = (uint16_t *)p; ctx->gemm_xs_elems = gx;
  }
  GemmScratch gs;
  gs.p = ctx->gemm_part; gs.floats = ctx->gemm_part_floats;
  gs.xs = ctx->gemm_xs; gs.xs_elems = ctx->gemm_xs_elems;
  return ctx_check(ctx, matmul(ctx->stream, m, (const float *)x->ptr, (float *)y->ptr, stride, row_base, input_offset, batch, &gs), "matmul");
}

uint64_t wgd_quantized_bytes(uint32_t cols) { return qx_bytes(cols); }

int wgd_quantize(wgd_context *ctx, const wgd_buffer *x, uint32_t cols, const wgd_buffer *norm_weight, float epsilon,
                 wgd_buffer *qx) {
  NEED_CTX(ctx); NEED_BUF(ctx, x, "quantize"); NEED_BUF(ctx, qx, "quantize");
  if (!cols) return fail(ctx, WGD_E_INVALID, "quantize: 0 columns");
  NEED_FIT(ctx, x, (uint64_t)cols * 4, "quantize input");
  NEED_FIT(ctx, qx, qx_bytes(cols), "quantized activation");
  if (norm_weight) { NEED_BUF(ctx, norm_weight, "quantize"); NEED_FIT(ctx, norm_weight, (uint64_t)cols * 4, "norm weight"); }
  int rc = ctx_check(ctx, quantize(ctx->stream, (const float *)x->ptr, cols, norm_weight ? (const float *)norm_weight->ptr : nullptr,
                                    qx_view(qx->ptr, cols)), "quantize");
  if (rc) return rc;
  qx->qx_cols = cols;
  qx->qx_normed = norm_weight != nullptr;
  qx->qx_eps = epsilon;
  return WGD_OK;
}

int wgd_matvec(wgd_context *ctx, int32_t type, const wgd_buffer *w, const wgd_buffer *qx, wgd_buffer *y, uint32_t cols,
               uint32_t rows, uint32_t row_base) {
  NEED_CTX(ctx); NEED_BUF(ctx, w, "matvec"); NEED_BUF(ctx, qx, "matvec"); NEED_BUF(ctx, y, "matvec");
  if (!known_type(type) || !cols || cols % block_size(type)) return fail(ctx, WGD_E_INVALID, "matvec: type %d, %u columns", type, cols);
  if (!rows) return WGD_OK;
  NEED_FIT(ctx, w, (uint64_t)rows * row_bytes(type, cols), "matvec weights");
  NEED_FIT(ctx, qx, qx_bytes(cols), "quantized activation");
  NEED_FIT(ctx, y, ((uint64_t)row_base + rows) * 4, "matvec output");
  Matrix m; m.data = (const uint8_t *)w->ptr; m.type = type; m.layout = w->layout; m.cols = cols; m.rows = rows;
  if (w->layout != LAYOUT_GGUF && (w->type != type || w->cols != cols || w->rows != rows))
    return fail(ctx, WGD_E_INVALID, "matvec: weights %s were uploaded as type %d, %ux%u", w->label.c_str(), w->type, w->cols, w->rows);
  if (!mv_supported(m)) return fail(ctx, WGD_E_INVALID, "matvec: type %d in this layout has no quantized matvec (upload with wgd_upload_weights)", type);
  if (qx->qx_cols != cols) return fail(ctx, WGD_E_INVALID, "matvec: %s holds no quantized row of %u columns (wgd_quantize first)", qx->label.c_str(), cols);
  const QXView xv = qx_const(qx_view(qx->ptr, cols), cols, qx->qx_normed, qx->qx_eps);
  return ctx_check(ctx, mv(ctx->stream, m, nullptr, xv, (float *)y->ptr + row_base, MV_STORE), "matvec");
}

int wgd_matvec_shapes(wgd_context *ctx, int32_t type, const wgd_buffer *w, const wgd_buffer *qx, wgd_buffer *y,
                      uint32_t cols, uint32_t rows, uint32_t max_shapes, uint32_t *count) {
  NEED_CTX(ctx); NEED_BUF(ctx, w, "matvec_shapes"); NEED_BUF(ctx, qx, "matvec_shapes"); NEED_BUF(ctx, y, "matvec_shapes");
  if (!count) return fail(ctx, WGD_E_INVALID, "matvec_shapes: NULL count");
  *count = 0;
  if (!known_type(type) || !cols || !rows || cols % block_size(type)) return fail(ctx, WGD_E_INVALID, "matvec_shapes: type %d, %ux%u", type, cols, rows);
  NEED_FIT(ctx, w, (uint64_t)rows * row_bytes(type, cols), "matvec weights");
  NEED_FIT(ctx, qx, qx_bytes(cols), "quantized activation");
  NEED_FIT(ctx, y, (uint64_t)max_shapes * rows * 4, "matvec_shapes output");
  Matrix m; m.data = (const uint8_t *)w->ptr; m.type = type; m.layout = w->layout; m.cols = cols; m.rows = rows;
  if (w->layout != LAYOUT_GGUF && (w->type != type || w->cols != cols || w->rows != rows))
    return fail(ctx, WGD_E_INVALID, "matvec_shapes: weights %s were uploaded as type %d, %ux%u", w->label.c_str(), w->type, w->cols, w->rows);
  if (!mv_supported(m)) return fail(ctx, WGD_E_INVALID, "matvec_shapes: type %d in this layout has no quantized matvec", type);
  if (qx->qx_cols != cols) return fail(ctx, WGD_E_INVALID, "matvec_shapes: %s holds no quantized row of %u columns", qx->label.c_str(), cols);
  const QXView xv = qx_const(qx_view(qx->ptr, cols), cols, qx->qx_normed, qx->qx_eps);
  return ctx_check(ctx, mv_shapes(ctx->stream, m, xv, (float *)y->ptr, max_shapes, count), "matvec_shapes");
}

int wgd_dequant(wgd_context *ctx, int32_t type, const wgd_buffer *w, wgd_buffer *out, uint64_t count) {
  NEED_CTX(ctx); NEED_BUF(ctx, w, "dequant"); NEED_BUF(ctx, out, "dequant");
  if (!known_type(type)) return fail(ctx, WGD_E_INVALID, "Unsupported quantization %d.", type);
  uint64_t bs = block_size(type);
  if (w->layout != LAYOUT_GGUF) return fail(ctx, WGD_E_INVALID, "dequant: %s holds repacked weights", w->label.c_str());
  NEED_FIT(ctx, w, (count + bs - 1) / bs * block_bytes(type), "dequant weights");
  NEED_FIT(ctx, out, count * 4, "dequant output");
  return ctx_check(ctx, dequant(ctx->stream, type, (const uint8_t *)w->ptr, (float *)out->ptr, count), "dequant");
}

int wgd_norm(wgd_context *ctx, const wgd_buffer *x, const wgd_buffer *w, wgd_buffer *y, uint32_t n, float eps, uint32_t batch) {
  NEED_CTX(ctx); NEED_BUF(ctx, x, "norm"); NEED_BUF(ctx, w, "norm"); NEED_BUF(ctx, y, "norm");
  NEED_FIT(ctx, x, (uint64_t)n * batch * 4, "norm input"); NEED_FIT(ctx, w, (uint64_t)n * 4, "norm weight");
  NEED_FIT(ctx, y, (uint64_t)n * batch * 4, "norm output");
  return ctx_check(ctx, norm(ctx->stream, (const float *)x->ptr, (const float *)w->ptr, (float *)y->ptr, n, eps, batch), "norm");
}

static int rope_common(wgd_context *ctx, wgd_buffer *x, const wgd_buffer *w, uint32_t heads, uint32_t hd, uint32_t start,
                       float theta, float scale, float eps, uint32_t rot, uint32_t batch, int mode) {
  NEED_BUF(ctx, x, "rope");
  if (hd == 0 || hd % 2 || rot % 2 || rot > hd) return fail(ctx, WGD_E_INVALID, "rope: head_dim %u / rotary_dim %u invalid", hd, rot);
  NEED_FIT(ctx, x, (uint64_t)heads * hd * batch * 4, "rope input");
  if (mode == 0) { NEED_BUF(ctx, w, "rope"); NEED_FIT(ctx, w, (uint64_t)hd * 4, "rope norm weight"); }
  return ctx_check(ctx, rope(ctx->stream, (float *)x->ptr, mode == 0 ? (const float *)w->ptr : nullptr, heads, hd, start, nullptr,
                             theta, scale, eps, rot, batch, mode), "rope");
}

int wgd_rope_norm(wgd_context *ctx, wgd_buffer *x, const wgd_buffer *w, uint32_t heads, uint32_t hd, uint32_t start,
                  float theta, float scale, float eps, uint32_t rot, uint32_t batch) {
  NEED_CTX(ctx);
  return rope_common(ctx, x, w, heads, hd, start, theta, scale, eps, rot, batch, 0);
}
int wgd_rope_neox(wgd_context *ctx, wgd_buffer *x, uint32_t heads, uint32_t hd, uint32_t start, float theta, float scale,
                  uint32_t rot, uint32_t batch) {
  NEED_CTX(ctx);
  return rope_common(ctx, x, nullptr, heads, hd, start, theta, scale, 0.f, rot, batch, 1);
}
int wgd_rope_adjacent(wgd_context *ctx, wgd_buffer *x, uint32_t heads, uint32_t hd, uint32_t start, float theta, float scale,
                      uint32_t rot, uint32_t batch) {
  NEED_CTX(ctx);
  return rope_common(ctx, x, nullptr, heads, hd, start, theta, scale, 0.f, rot, batch, 2);
}

// The checks and arguments shared by both attention entry points (partial left unset).
static int attention_args(wgd_context *ctx, const char *what, const wgd_buffer *q, const wgd_buffer *k,
                          const wgd_buffer *v, wgd_buffer *y, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                          uint32_t start, float scale, uint32_t window, uint32_t capacity, uint32_t context,
                          uint32_t batch, AttnArgs &a, bool kv16 = false) {
  NEED_BUF(ctx, q, what); NEED_BUF(ctx, k, what); NEED_BUF(ctx, v, what); NEED_BUF(ctx, y, what);
  const uint64_t esz = kv16 ? 2 : 4;  // bytes per ring element
  uint32_t cap = capacity ? capacity : context;
  if (!kv_heads || !heads || heads % kv_heads || !hd || hd > 512 || !cap || !window)
    return fail(ctx, WGD_E_INVALID, "%s: invalid heads %u/%u, head_dim %u, capacity %u or window %u", what, heads, kv_heads, hd, cap, window);
  if ((heads / kv_heads) > 16) return fail(ctx, WGD_E_INVALID, "%s: more than 16 query heads per KV head", what);
  NEED_FIT(ctx, q, (uint64_t)batch * heads * hd * 4, "attention queries");
  NEED_FIT(ctx, k, (uint64_t)cap * kv_heads * hd * esz, "attention keys");
  NEED_FIT(ctx, v, (uint64_t)cap * kv_heads * hd * esz, "attention values");
  NEED_FIT(ctx, y, (uint64_t)batch * heads * hd * 4, "attention output");
  a = AttnArgs{};
  a.q = (const float *)q->ptr; a.k = k->ptr; a.v = v->ptr; a.y = (float *)y->ptr;
  a.kv16 = kv16;
  a.heads = heads; a.kv_heads = kv_heads; a.hd = hd; a.start = start; a.start_dev = nullptr;
  a.scale = scale; a.window = window; a.capacity = cap; a.batch = batch;
  a.partial = nullptr; a.partial_floats = 0;
  return WGD_OK;
}

static int attention_common(wgd_context *ctx, const char *what, const wgd_buffer *q, const wgd_buffer *k,
                            const wgd_buffer *v, wgd_buffer *y, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                            uint32_t start, float scale, uint32_t window, uint32_t capacity, uint32_t context,
                            uint32_t batch, bool kv16) {
  NEED_CTX(ctx);
  AttnArgs a;
  int rc = attention_args(ctx, what, q, k, v, y, heads, kv_heads, hd, start, scale, window, capacity, context, batch, a, kv16);
  if (rc || !batch) return rc;
  uint64_t need = attention_scratch_floats(heads, hd, batch, (uint32_t)device_cu_count() * 4);
  if (need > ctx->att_partial_floats) {
    ctx_free(ctx, ctx->att_partial);
    ctx->att_partial = nullptr; ctx->att_partial_floats = 0;
    void *p = nullptr;
    rc = ctx_alloc(ctx, need * 4, "attention split scratch", &p);
    if (rc) return rc;
    ctx->att_partial = (float *)p; ctx->att_partial_floats = need;
  }
  a.partial = ctx->att_partial; a.partial_floats = (uint32_t)(ctx->att_partial_floats > 0xFFFFFFFFull ? 0xFFFFFFFFull : ctx->att_partial_floats);
  return ctx_check(ctx, attention(ctx->stream, a), what);
}

int wgd_attention(wgd_context *ctx, const wgd_buffer *q, const wgd_buffer *k, const wgd_buffer *v, wgd_buffer *y,
                  uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t start, float scale, uint32_t window,
                  uint32_t capacity, uint32_t context, uint32_t batch) {
  return attention_common(ctx, "attention", q, k, v, y, heads, kv_heads, hd, start, scale, window, capacity, context,
                          batch, false);
}

int wgd_attention_f16kv(wgd_context *ctx, const wgd_buffer *q, const wgd_buffer *k, const wgd_buffer *v,
                        wgd_buffer *y, uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t start, float scale,
                        uint32_t window, uint32_t capacity, uint32_t context, uint32_t batch) {
  return attention_common(ctx, "attention_f16kv", q, k, v, y, heads, kv_heads, hd, start, scale, window, capacity,
                          context, batch, true);
}

int wgd_kv_store_f16(wgd_context *ctx, const wgd_buffer *src, wgd_buffer *dst, uint64_t count, uint64_t src_offset,
                     uint64_t dst_offset) {
  NEED_CTX(ctx); NEED_BUF(ctx, src, "kv_store_f16"); NEED_BUF(ctx, dst, "kv_store_f16");
  if (src_offset > src->size / 4 || count > src->size / 4 - src_offset || dst_offset > dst->size / 2 ||
      count > dst->size / 2 - dst_offset)
    return fail(ctx, WGD_E_INVALID, "kv_store_f16: %llu values from float %llu of a %llu-byte buffer into half %llu of a "
                "%llu-byte buffer overrun", (unsigned long long)count, (unsigned long long)src_offset,
                (unsigned long long)src->size, (unsigned long long)dst_offset, (unsigned long long)dst->size);
  return ctx_check(ctx, to_f16(ctx->stream, (const float *)src->ptr + src_offset, (_Float16 *)dst->ptr + dst_offset, count),
                   "kv_store_f16");
}

int wgd_probe_read(wgd_context *ctx, const wgd_buffer *src, uint64_t bytes, uint32_t copies, uint32_t launches,
                   uint32_t workgroups, uint32_t threads, uint32_t depth, wgd_buffer *out, uint32_t out_floats) {
  NEED_CTX(ctx); NEED_BUF(ctx, src, "probe_read");
  const uint64_t stride = (bytes + 4095) / 4096 * 4096;
  if (!bytes || bytes % 16 || bytes >= (1ull << 31) || !copies || !launches || copies * stride > src->size || !workgroups ||
      !threads || threads % 64 || threads > 1024 || (depth != 4 && depth != 8 && depth != 16))
    return fail(ctx, WGD_E_INVALID, "probe_read: %llu bytes (multiple of 16, < 2 GiB) x %u copies within the buffer, "
                "%u launches, %u workgroups of %u threads (multiple of 64, <= 1024), depth %u (4, 8 or 16)",
                (unsigned long long)bytes, copies, launches, workgroups, threads, depth);
  if (out_floats) {
    NEED_BUF(ctx, out, "probe_read");
    NEED_FIT(ctx, out, (uint64_t)out_floats * 4, "probe_read output");
  }
  for (uint32_t i = 0; i < launches; i++) {
    const uint8_t *p = (const uint8_t *)src->ptr + (uint64_t)(i % copies) * stride;
    int rc = ctx_check(ctx, probe_read(ctx->stream, p, (uint32_t)bytes, workgroups, threads, depth,
                                       out ? (float *)out->ptr : nullptr, out_floats), "probe_read");
    if (rc) return rc;
  }
  return WGD_OK;
}

// ---------------------------------------------------------------- allocation-free attention
// The split-K partials of wgd_attention_noalloc live in this array of the library's own
// device memory: each GPU the library runs on holds one copy until the process ends, so the
// entry point calls no allocator. In host code `scratch` names a host-side stand-in, never
// device memory: its address on each GPU comes from hipGetSymbolAddress, taken once per
// device by wgd_create with that device current, and only that address reaches kernels.
// Calls on one GPU share its copy (overlapping calls from two streams race); every split
// writes each of its partial rows before the merge reads them, so nothing needs clearing.
static constexpr uint64_t NOALLOC_SCRATCH_FLOATS = 8ull << 20;  // 32 MiB
static __device__ __attribute__((used)) __align__(256) float scratch[NOALLOC_SCRATCH_FLOATS];
static constexpr int SCRATCH_DEVICES = 64;
static std::mutex g_scratch_mu;
static float *g_scratch_ptr[SCRATCH_DEVICES];

// The device address of `scratch` on the current device `device` (once per device).
static int scratch_setup(int device, float **out) {
  if (device < 0 || device >= SCRATCH_DEVICES)
    return fail(nullptr, WGD_E_DEVICE, "device %d is beyond the %d devices the static scratch covers", device, SCRATCH_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(nullptr, WGD_E_DEVICE, "static scratch address on device %d: %s", device, hipGetErrorString(e));
    g_scratch_ptr[device] = (float *)ptr;
  }
  *out = g_scratch_ptr[device];
  return WGD_OK;
}

int wgd_attention_noalloc(wgd_context *ctx, const wgd_buffer *q, const wgd_buffer *k, const wgd_buffer *v,
                          wgd_buffer *y, uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t start, float scale,
                          uint32_t window, uint32_t capacity, uint32_t context, uint32_t batch) {
  NEED_CTX(ctx);
  AttnArgs a;
  int rc = attention_args(ctx, "attention_noalloc", q, k, v, y, heads, kv_heads, hd, start, scale, window, capacity,
                          context, batch, a);
  if (rc || !batch) return rc;
  if (!ctx->noalloc_scratch) return fail(ctx, WGD_E_STATE, "attention_noalloc: no static scratch on device %d", ctx->device);
  // the split plan of wgd_attention, whose scratch never limits it: the same launches and
  // the same partial sums, so both entry points give the same bits
  const uint64_t need = attention_partial_need(a);
  if (need > NOALLOC_SCRATCH_FLOATS)
    return fail(ctx, WGD_E_INVALID,
                "attention_noalloc: %u tokens x %u heads x head_dim %u need %llu floats of split scratch; the static "
                "scratch holds %llu (use wgd_attention or a smaller batch)",
                batch, heads, hd, (unsigned long long)need, (unsigned long long)NOALLOC_SCRATCH_FLOATS);
  a.partial = ctx->noalloc_scratch;
  a.partial_floats = (uint32_t)need;
  return ctx_check(ctx, attention(ctx->stream, a), "attention_noalloc");
}

uint64_t wgd_attention_noalloc_limit(void) { return NOALLOC_SCRATCH_FLOATS; }

int wgd_add(wgd_context *ctx, const wgd_buffer *delta, wgd_buffer *state, uint32_t n) {
  NEED_CTX(ctx); NEED_BUF(ctx, delta, "add"); NEED_BUF(ctx, state, "add");
  NEED_FIT(ctx, delta, (uint64_t)n * 4, "add delta"); NEED_FIT(ctx, state, (uint64_t)n * 4, "add state");
  return ctx_check(ctx, add(ctx->stream, (const float *)delta->ptr, (float *)state->ptr, n), "add");
}

static int glu_common(wgd_context *ctx, const wgd_buffer *g, const wgd_buffer *u, wgd_buffer *y, uint32_t n, int act) {
  NEED_CTX(ctx); NEED_BUF(ctx, g, "glu"); NEED_BUF(ctx, u, "glu"); NEED_BUF(ctx, y, "glu");
  NEED_FIT(ctx, g, (uint64_t)n * 4, "glu gate"); NEED_FIT(ctx, u, (uint64_t)n * 4, "glu up"); NEED_FIT(ctx, y, (uint64_t)n * 4, "glu output");
  return ctx_check(ctx, glu(ctx->stream, (const float *)g->ptr, (const float *)u->ptr, (float *)y->ptr, n, act), "glu");
}
int wgd_silu(wgd_context *ctx, const wgd_buffer *g, const wgd_buffer *u, wgd_buffer *y, uint32_t n) { return glu_common(ctx, g, u, y, n, 0); }
int wgd_gelu(wgd_context *ctx, const wgd_buffer *g, const wgd_buffer *u, wgd_buffer *y, uint32_t n) { return glu_common(ctx, g, u, y, n, 1); }

int wgd_bias_add(wgd_context *ctx, wgd_buffer *y, const wgd_buffer *b, uint32_t n, uint32_t width) {
  NEED_CTX(ctx); NEED_BUF(ctx, y, "bias"); NEED_BUF(ctx, b, "bias");
  if (!width) return fail(ctx, WGD_E_INVALID, "bias: width 0");
  NEED_FIT(ctx, y, (uint64_t)n * 4, "bias target"); NEED_FIT(ctx, b, (uint64_t)(n < width ? n : width) * 4, "bias vector");
  return ctx_check(ctx, bias_add(ctx->stream, (float *)y->ptr, (const float *)b->ptr, n, width), "bias");
}

int wgd_activate(wgd_context *ctx, wgd_buffer *x, uint32_t n) {
  NEED_CTX(ctx); NEED_BUF(ctx, x, "activate");
  NEED_FIT(ctx, x, (uint64_t)n * 4, "activate");
  return ctx_check(ctx, activate(ctx->stream, (float *)x->ptr, n), "activate");
}

int wgd_argmax(wgd_context *ctx, const wgd_buffer *logits, uint32_t n, wgd_buffer *out, int32_t *host_index) {
  NEED_CTX(ctx); NEED_BUF(ctx, logits, "argmax");
  NEED_FIT(ctx, logits, (uint64_t)n * 4, "argmax logits");
  if (out) { NEED_BUF(ctx, out, "argmax"); NEED_FIT(ctx, out, 4, "argmax output"); }
  int rc = ctx_check(ctx, argmax(ctx->stream, (const float *)logits->ptr, n, ctx->argmax_scratch), "argmax");
  if (rc) return rc;
  if (out) {
    rc = ctx_check(ctx, hipMemcpyAsync(out->ptr, ctx->argmax_scratch, 4, hipMemcpyDeviceToDevice, ctx->stream), "argmax");
    if (rc) return rc;
  }
  if (host_index) {
    rc = ctx_sync(ctx, "argmax");
    if (rc) return rc;
    int32_t id = -1;
    hipError_t e = hipMemcpy(&id, ctx->argmax_scratch, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(ctx, e, "argmax read-back");
    *host_index = id;
    if (id < 0) return fail(ctx, WGD_E_NONFINITE, "Inference produced non-finite logits. Stop and report this model/runtime combination.");
  }
  return WGD_OK;
}

int wgd_sample(wgd_context *ctx, const wgd_buffer *logits, uint32_t n, double temperature, uint32_t top_k,
               double top_p, uint64_t seed, uint32_t index, int32_t *token) {
  NEED_CTX(ctx); NEED_BUF(ctx, logits, "sample");
  NEED_FIT(ctx, logits, (uint64_t)n * 4, "sample logits");
  if (!token || !n || index > 0x7FFFFFFFu) return fail(ctx, WGD_E_INVALID, "wgd_sample: bad arguments");
  if (!(temperature >= 0.0 && temperature <= 2.0) || top_k < 1 || top_k > 200 || !(top_p > 0.0 && top_p <= 1.0))
    return fail(ctx, WGD_E_INVALID, "Invalid sampling settings.");
  if (!ctx->sample_params) {
    int rc = ctx_alloc(ctx, sizeof(SampleParams), "sampling settings", (void **)&ctx->sample_params);
    if (rc) return rc;
  }
  const SampleParams p = {temperature, top_p, top_k, 0, seed};
  int rc = ctx_check(ctx, hipMemcpyAsync(ctx->sample_params, &p, sizeof p, hipMemcpyHostToDevice, ctx->stream), "sample");
  if (!rc && ctx->sample_scratch_bytes < sample_scratch_bytes(n)) {
    if (ctx->sample_scratch) ctx_free(ctx, ctx->sample_scratch);
    ctx->sample_scratch = nullptr;
    ctx->sample_scratch_bytes = 0;
    rc = ctx_alloc(ctx, sample_scratch_bytes(n), "sampling candidates", &ctx->sample_scratch);
    if (!rc) ctx->sample_scratch_bytes = sample_scratch_bytes(n);
  }
  if (!rc) rc = ctx_check(ctx, sample(ctx->stream, (const float *)logits->ptr, n, ctx->sample_params, (int32_t)index,
                                      nullptr, ctx->argmax_scratch, nullptr, 0, false, ctx->sample_scratch), "sample");
  if (!rc) rc = ctx_sync(ctx, "sample");
  if (rc) return rc;
  int32_t id = -1;
  hipError_t e = hipMemcpy(&id, ctx->argmax_scratch, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(ctx, e, "sample read-back");
  *token = id;
  if (id < 0) return fail(ctx, WGD_E_NONFINITE, "Inference produced non-finite logits. Stop and report this model/runtime combination.");
  return WGD_OK;
}

int wgd_embed(wgd_context *ctx, int32_t type, const wgd_buffer *table, const wgd_buffer *ids, wgd_buffer *out,
              uint32_t hidden, uint32_t n, double scale) {
  NEED_CTX(ctx); NEED_BUF(ctx, table, "embed"); NEED_BUF(ctx, ids, "embed"); NEED_BUF(ctx, out, "embed");
  if (!known_type(type) || hidden % block_size(type)) return fail(ctx, WGD_E_INVALID, "embed: bad type %d or hidden %u", type, hidden);
  NEED_FIT(ctx, ids, (uint64_t)n * 4, "embed ids"); NEED_FIT(ctx, out, (uint64_t)n * hidden * 4, "embed output");
  uint64_t rb = row_bytes(type, hidden), rows = table->size / rb;
  // Row ids come from the host: check them before they index the table.
  if (n) {
    int rc = ctx_sync(ctx, "embed");
    if (rc) return rc;
    std::string tmp(n * 4, '\0');
    hipError_t e = hipMemcpy(&tmp[0], ids->ptr, n * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(ctx, e, "embed ids");
    for (uint32_t i = 0; i < n; i++) {
      int32_t id; memcpy(&id, tmp.data() + 4 * i, 4);
      if (id < 0 || (uint64_t)id >= rows) return fail(ctx, WGD_E_INVALID, "embed: token id %d outside the %llu-row table", id, (unsigned long long)rows);
    }
  }
  Matrix t; t.data = (const uint8_t *)table->ptr; t.type = type; t.cols = hidden; t.rows = (uint32_t)rows;
  if (table->layout != LAYOUT_GGUF) {
    if (table->type != type || table->cols != hidden) return fail(ctx, WGD_E_INVALID, "embed: table %s has another type or width", table->label.c_str());
    t.layout = table->layout; t.rows = table->rows;
  }
  return ctx_check(ctx, embed_matrix(ctx->stream, t, (const int32_t *)ids->ptr, (float *)out->ptr, n, scale), "embed");
}

}  // extern "C"
