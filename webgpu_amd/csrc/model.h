// model.h — context and model state shared by runtime.hip and model.hip.
#pragma once
#include <map>
#include <set>
#include <string>
#include <vector>

#include "internal.h"

struct wgd_buffer;
struct wgd_model;

struct wgd_context {
  int device = 0;
  hipStream_t stream = nullptr;
  uint64_t limit = 0, allocated = 0, peak = 0;
  std::string error, adapter;
  std::set<wgd_buffer *> buffers;
  std::set<wgd_model *> models;
  std::map<void *, uint64_t> sizes;   // every device allocation of the context
  int32_t *argmax_scratch = nullptr;  // int32 result + 256 partial keys
  float *att_partial = nullptr;       // split-K scratch of the per-kernel attention launcher
  uint64_t att_partial_floats = 0;
  float *noalloc_scratch = nullptr;  // this device's static scratch (wgd_attention_noalloc)
  void *mv_qx = nullptr;              // quantized activation row of wgd_matmul
  uint64_t mv_qx_bytes = 0;
  float *gemm_part = nullptr;         // split-K partial sums of wgd_matmul's prompt GEMM
  uint64_t gemm_part_floats = 0;
  uint16_t *gemm_xs = nullptr;        // its input split into bf16 (hi, lo)
  uint64_t gemm_xs_elems = 0;
  wgd::SampleParams *sample_params = nullptr;  // settings of wgd_sample
  void *sample_scratch = nullptr;              // its slices' candidates
  uint64_t sample_scratch_bytes = 0;
};

namespace wgd {
int fail(wgd_context *ctx, int code, const char *fmt, ...);
int hip_fail(wgd_context *ctx, hipError_t e, const char *what);
int ctx_alloc(wgd_context *ctx, uint64_t size, const char *label, void **out);
void ctx_free(wgd_context *ctx, void *p);
int ctx_check(wgd_context *ctx, hipError_t launch, const char *what);
int ctx_sync(wgd_context *ctx, const char *what);
void model_destroy(wgd_model *m);
// Embedding gather from a GGUF or planar table.
hipError_t embed_matrix(hipStream_t s, const Matrix &table, const int32_t *ids, float *out, uint32_t n,
                        double scale);
}  // namespace wgd
