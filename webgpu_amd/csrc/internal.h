// internal.h — shared declarations of libwgd (gfx950). Kernel launchers take raw device
// pointers and a stream; the C-ABI layer (runtime.hip) and the native decoder step
// (model.hip) both call them.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <string>

#include "../../include/wgd.h"

namespace wgd {

// GGUF quantization ids (gguf.ts:6-11).
enum QType : int { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14 };

inline int block_size(int t) {
  switch (t) { case F32: case F16: return 1; case Q4_0: case Q8_0: return 32;
    case Q4_K: case Q5_K: case Q6_K: return 256; }
  return 0;
}
inline int block_bytes(int t) {
  switch (t) { case F32: return 4; case F16: return 2; case Q4_0: return 18; case Q8_0: return 34;
    case Q4_K: return 144; case Q5_K: return 176; case Q6_K: return 210; }
  return 0;
}
inline uint64_t row_bytes(int t, uint64_t cols) { return cols / block_size(t) * block_bytes(t); }

// Device layouts of a weight matrix. GGUF keeps the file's block bytes. The planar
// layouts (Q4_K, Q6_K, Q8_0) hold the same bits rearranged for the decode matvec: the
// quants of each 32 consecutive elements of a row (16 for Q8_0) form a 16-byte "chunk"
// (C chunks per row), the per-block fields (Q4_K header, Q6_K high bits / scales / d,
// Q8_0 d) live in separate planes, and rows are grouped in tiles of 16: within a tile,
// the 16 rows' entries of one column are consecutive, so 16 rows x 4 columns of chunks
// are 1 KB of contiguous bytes. Rows are padded to a multiple of 16 (zero bytes).
enum Layout : int { LAYOUT_GGUF = 0, LAYOUT_PLANAR = 1 };

struct Matrix {
  const uint8_t *data = nullptr;
  int type = F32;
  int layout = LAYOUT_GGUF;
  uint32_t cols = 0, rows = 0;
};

// Entry (row, col) of a tiled plane with ncols columns.
__host__ __device__ inline uint64_t tiled(uint64_t row, uint64_t col, uint64_t ncols) {
  return ((row >> 4) * ncols + col) * 16 + (row & 15);
}
__host__ __device__ inline uint64_t tile_rows(uint64_t rows) { return (rows + 15) / 16 * 16; }
// Plane offsets for nbp blocks (padded rows x blocks per row).
struct Q4Planes { uint64_t qs, hdr; };
__host__ __device__ inline Q4Planes q4_planes(uint64_t nbp) { return {0, nbp * 128}; }
struct Q6Planes { uint64_t ql, qh, sc, d; };
__host__ __device__ inline Q6Planes q6_planes(uint64_t nbp) { return {0, nbp * 128, nbp * 192, nbp * 208}; }
struct Q8Planes { uint64_t qs, d; };
__host__ __device__ inline Q8Planes q8_planes(uint64_t nbp) { return {0, nbp * 32}; }
// Q5_K: the Q4_K nibble chunks, one dword of fifth bits per chunk, the 16-byte header.
struct Q5Planes { uint64_t qs, qh, hdr; };
__host__ __device__ inline Q5Planes q5_planes(uint64_t nbp) { return {0, nbp * 128, nbp * 160}; }
// Q4_0: a block is one chunk; its 16 quant bytes, then d per block.
struct Q40Planes { uint64_t qs, d; };
__host__ __device__ inline Q40Planes q40_planes(uint64_t nbp) { return {0, nbp * 16}; }
__host__ __device__ inline uint32_t chunk_elems(int type) { return type == Q8_0 ? 16u : 32u; }

// Whether matrices of this type and width are stored in the planar layout: the K-quants,
// and Q8_0 / Q4_0 in whole 64-column tiles (the prompt GEMM's K tile).
bool has_planar(int type, uint64_t cols);
// Bytes of a planar matrix (rows padded to 16).
uint64_t planar_bytes(int type, uint32_t cols, uint32_t rows);
// Rewrites a GGUF matrix (rows x cols) into the planar layout (device to device); dst must
// hold planar_bytes and be zero-filled (padding rows).
hipError_t repack_planar(hipStream_t s, int type, const uint8_t *src, uint8_t *dst, uint32_t cols, uint32_t rows);

// ---------------------------------------------------------------- launchers

// Scratch of the prompt GEMM on planar weights. p: split-K partial sums, of which
// gemm_split_floats() is what a launch of w over `batch` tokens can use (0: it does not
// split; less scratch means fewer splits). xs: the activations split into bf16 (hi, lo) in
// MFMA fragment order, gemm_input_elems() of them (without it the generic kernel runs).
// xs_of/xs_cols/xs_batch name the activations xs holds, so GEMMs over the same input split
// it once; whoever rewrites that memory clears xs_of.
struct GemmScratch {
  float *p = nullptr; uint64_t floats = 0;
  uint16_t *xs = nullptr; uint64_t xs_elems = 0;
  const float *xs_of = nullptr; uint32_t xs_cols = 0, xs_batch = 0;
};
uint64_t gemm_split_floats(const Matrix &w, uint32_t batch);
uint64_t gemm_input_elems(uint32_t cols, uint32_t batch);
// True when a GEMM of w over `batch` tokens runs the planar-weight kernel on the split input
// (and may add into y).
bool gemm_splits_input(const Matrix &w, const GemmScratch *scratch, uint32_t batch);

// Up to three planar matrices with the same columns (at most two weight types) that read
// the same activations, in one launch: y_j[b*stride_j + row_base_j + r] = W_j x_b, or
// += with accumulate. glu_out (two jobs of equal rows: gate, up): act(gate) * up is written
// there, [batch][rows], and its split into scratch->xs for the GEMM that reads it; the
// jobs' own y are not written.
struct GemmJob { const Matrix *w = nullptr; float *y = nullptr; uint32_t stride = 0, row_base = 0; };
// An RMSNorm left to the consumer of a GEMM: the GEMM's input was the split of x * w (the
// norm weight) and the products are scaled per token by 1 / sqrt(sum(x^2) / n + eps), the
// token's sum of squares being sq[tok * segs + 0 .. segs) added in that order. sq == null:
// the input was normed already.
struct DeferredNorm { const float *sq = nullptr; uint32_t segs = 0, n = 0; float eps = 0.f; };
#ifdef __HIPCC__
__device__ __forceinline__ float deferred_inv(const DeferredNorm &d, uint32_t tok) {
  if (!d.sq) return 1.f;
  float t = 0.f;
  for (uint32_t u = 0; u < d.segs; u++) t += d.sq[(uint64_t)tok * d.segs + u];
  return 1.f / sqrtf(t / (float)d.n + d.eps);
}
#endif
struct GemmGroup {
  GemmJob job[3]; uint32_t n = 0;
  bool accumulate = false;
  float *glu_out = nullptr; int glu_act = 0;
  // the GLU finish also stores glu_out in f32 (off when only its split is read next)
  bool glu_f32 = true;
  DeferredNorm glu_norm;  // the input's pending RMSNorm, applied to gate and up in the GLU finish
  // leave the split-K partials (one split too) in scratch->p for the caller's own finish;
  // the number of splits is returned in *splits
  bool keep_partials = false; uint32_t *splits = nullptr;
};
bool gemm_group_ok(const GemmGroup &g, uint32_t batch);

// Decode-loop state in device memory: the position and id of the token being fed, the
// step count, and a flag for a step whose logits had no finite entry.
struct StepState { int32_t pos, token, step, error; };
// Sampling settings of engine.ts:21 (temperature 0: greedy) and the seed of the uniforms
// that replace Math.random().
struct SampleParams { double temperature, top_p; uint32_t top_k, pad; uint64_t seed; };
// sample() of engine.ts:305-324 on logits[0..n): the token to *out, drawn with the index-th
// uniform of the seed (index < 0: st->pos + 1); with `advance`, recorded in st and
// tokens[st->step] and the position advanced, as the greedy step does. `scratch` holds
// sample_scratch_bytes(n) of device memory (the slices' candidates).
uint64_t sample_scratch_bytes(uint32_t n);
hipError_t sample(hipStream_t s, const float *logits, uint32_t n, const SampleParams *params, int32_t index,
                  StepState *st, int32_t *out, int32_t *tokens, uint32_t cap, bool advance, void *scratch);
uint64_t gemm_group_split_floats(const GemmGroup &g, uint32_t batch);
hipError_t gemm_group(hipStream_t s, const GemmGroup &g, const float *x, uint32_t batch, GemmScratch *scratch);
// y[b*stride + row_base + r] = sum_c deq(W)[r][c] * x[(b+input_offset)*cols + c]: the
// generic kernel for small batches of GGUF-layout weights, else the MFMA dequant-GEMM.
// accumulate (planar weights with split-input scratch only): y[...] += the sum.
hipError_t matmul(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                  uint32_t row_base, uint32_t input_offset, uint32_t batch, GemmScratch *scratch = nullptr,
                  bool accumulate = false);
hipError_t matmul_generic(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                          uint32_t row_base, uint32_t input_offset, uint32_t batch);
hipError_t gemm(hipStream_t s, const Matrix &w, const float *x, float *y, uint32_t stride,
                uint32_t row_base, uint32_t input_offset, uint32_t batch, GemmScratch *scratch = nullptr,
                bool accumulate = false);

hipError_t dequant(hipStream_t s, int type, const uint8_t *w, float *out, uint64_t count);
hipError_t embed(hipStream_t s, int type, const uint8_t *table, const int32_t *ids, float *out,
                 uint32_t hidden, uint32_t n, double scale);
hipError_t norm(hipStream_t s, const float *x, const float *w, float *y, uint32_t n, float eps,
                uint32_t batch);
// The deferred-norm form of reduce_norm_split: state += the partials (split order), xs = the
// split of state * w, and each token's sum of squares of state in residual_split_segs(n)
// segments to sq, for a consumer that applies the norm factor (DeferredNorm).
uint32_t residual_split_segs(uint32_t n);
hipError_t residual_split(hipStream_t s, const float *part, uint32_t splits, float *state, const float *w, uint16_t *xs,
                          float *sq, uint32_t n, uint32_t batch);
// Per token: state += the split-K partial sums part[z][tok][n] (in split order), then
// norm_split() of the new state into y and xs (n % 64 == 0, n <= 16384). With post_w the
// sums are a delta added as RMSNorm(delta) * post_w (Gemma's post-norms).
hipError_t reduce_norm_split(hipStream_t s, const float *part, uint32_t splits, float *state, const float *w, float *y,
                             uint16_t *xs, uint32_t n, float eps, uint32_t batch, const float *post_w = nullptr);
// norm() that also writes its output in the prompt GEMM's split form into xs (n % 64 == 0).
hipError_t norm_split(hipStream_t s, const float *x, const float *w, float *y, uint16_t *xs, uint32_t n, float eps,
                      uint32_t batch);
// mode 0: Q/K norm + half-split, 1: half-split, 2: adjacent pairs. start_dev overrides start.
hipError_t rope(hipStream_t s, float *x, const float *w, uint32_t heads, uint32_t hd,
                uint32_t start, const int32_t *start_dev, float theta, float scale, float eps,
                uint32_t rotary_dim, uint32_t batch, int mode);
// The finish of a Q/K/V GEMM group kept as split-K partials (rows q | k | v per token):
// sums, bias, RoPE (rope()'s modes), Q into q and K/V into ring slot (start + t) % capacity.
struct QKVFinish {
  const float *part = nullptr; uint32_t splits = 0, rows_total = 0, batch = 0;
  const float *bq = nullptr, *bk = nullptr, *bv = nullptr;
  const float *qn = nullptr, *kn = nullptr;  // mode 0 norm weights
  float *q = nullptr; void *kc = nullptr, *vc = nullptr; uint32_t capacity = 0;
  bool kv16 = false;  // ring elements are f16
  uint32_t heads = 0, kvh = 0, hd = 0, rot = 0, start = 0; const int32_t *start_dev = nullptr;
  float eps = 0.f; int mode = 1;
  const float2 *cs = nullptr;  // rope_table() of the batch's positions
  DeferredNorm xnorm;          // the GEMM input's pending RMSNorm, applied to the sums first
};
hipError_t qkv_finish(hipStream_t s, const QKVFinish &a);
// cs[t * rot/2 + i] = (cos, sin) of (start + t) * scale * theta^(-2i/rot) for t < n (angles in
// f64, as rope() forms them); start_dev overrides start.
hipError_t rope_table(hipStream_t s, float2 *cs, uint32_t rot, uint32_t n, uint32_t start, const int32_t *start_dev,
                      float theta, float scale);
struct AttnArgs {
  const float *q; const void *k; const void *v; float *y;  // k, v: the K/V ring (f32, or f16 with kv16)
  uint32_t heads, kv_heads, hd, start; const int32_t *start_dev;
  float scale; uint32_t window, capacity, batch;
  float *partial; uint32_t partial_floats;  // split-K scratch (may be null: single split)
  // optional: the output also in the prompt GEMM's split form; *xs_written says whether it was
  uint16_t *xs = nullptr; bool *xs_written = nullptr;
  bool kv16 = false;
};
hipError_t attention(hipStream_t s, const AttnArgs &a);
// Floats of split-K partials attention() writes for these arguments when its scratch does
// not limit the split count (0: one split, no scratch used).
uint64_t attention_partial_need(const AttnArgs &a);
uint64_t attention_scratch_floats(uint32_t heads, uint32_t hd, uint32_t batch, uint32_t max_keys);
hipError_t add(hipStream_t s, const float *delta, float *state, uint32_t n);
hipError_t glu(hipStream_t s, const float *gate, const float *up, float *y, uint32_t n, int act);
// glu() over [batch][cols] that also writes y in the prompt GEMM's split form (cols % 64 == 0).
hipError_t glu_split(hipStream_t s, const float *gate, const float *up, float *y, uint16_t *xs, uint32_t cols,
                     uint32_t batch, int act);
hipError_t bias_add(hipStream_t s, float *y, const float *b, uint32_t n, uint32_t width);
hipError_t activate(hipStream_t s, float *x, uint32_t n);
// argmax over finite values, first index wins; writes -1 when none is finite.
hipError_t argmax(hipStream_t s, const float *logits, uint32_t n, int32_t *out);
// Copies K/V rows of a batch into ring slots (start + i) % capacity; an f16 ring (kv16)
// stores each value rounded to the nearest f16 (ties to even).
hipError_t kv_append(hipStream_t s, const float *k, const float *v, void *kc, void *vc,
                     uint32_t row_floats, uint32_t n, uint32_t start, const int32_t *start_dev,
                     uint32_t capacity, bool kv16 = false);
// n f32 values of src into an f16 buffer, rounded to nearest (ties to even).
hipError_t to_f16(hipStream_t s, const float *src, _Float16 *dst, uint64_t n);

#ifdef __HIPCC__
// K/V ring elements: f32, or f16 (stored rounded to nearest even, widened exactly on load).
template <class E> __device__ __forceinline__ float kv_get(const void *ring, uint64_t i) {
  return (float)((const E *)ring)[i];
}
template <class E> __device__ __forceinline__ float4 kv_get4(const void *ring, uint64_t i) {
  if constexpr (sizeof(E) == 4) return *(const float4 *)((const float *)ring + i);
  const uint2 h = *(const uint2 *)((const _Float16 *)ring + i);
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 a = __builtin_bit_cast(h2, h.x), b = __builtin_bit_cast(h2, h.y);
  return make_float4((float)a.x, (float)a.y, (float)b.x, (float)b.y);
}
__device__ __forceinline__ void kv_put(void *ring, uint64_t i, float x, bool f16) {
  if (f16) ((_Float16 *)ring)[i] = (_Float16)x;
  else ((float *)ring)[i] = x;
}
template <class E> __device__ __forceinline__ void kv_put4(void *ring, uint64_t i, const float4 &v) {
  if constexpr (sizeof(E) == 4) {
    *(float4 *)((float *)ring + i) = v;
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 a = {(_Float16)v.x, (_Float16)v.y}, b = {(_Float16)v.z, (_Float16)v.w};
    *(uint2 *)((_Float16 *)ring + i) = make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
  }
}
#endif
// Normalise `delta` with w (post-norm) and add into state: state += norm(delta) * w.
hipError_t norm_add(hipStream_t s, const float *delta, const float *w, float *state, uint32_t n,
                    float eps, uint32_t batch);

int device_cu_count();
// A plain streaming read of bytes (multiple of 16) by wgs workgroups of `threads`, depth
// 16-byte loads in flight per lane; out_n > 0 also stores an out_n-float result.
hipError_t probe_read(hipStream_t s, const uint8_t *p, uint32_t bytes, uint32_t wgs, uint32_t threads, uint32_t depth,
                      float *out, uint32_t out_n);
// Lets `kernel` take dynamic LDS up to the CU's 160 KB (the default limit is 64 KB): set
// once per kernel (each template instance is its own kernel), before its first launch.
void lds_opt_in(const void *kernel);
constexpr uint32_t LDS_MAX = 160 * 1024;

}  // namespace wgd

#define WGD_HIP(expr)                         \
  do {                                        \
    hipError_t _e = (expr);                   \
    if (_e != hipSuccess) return _e;          \
  } while (0)
