/*
 * wgd.h — C ABI of the MI355X (gfx950) dense-decoder library `libwgd.so`.
 *
 * This boundary replaces the WebGPU layer of ahpah-dev/WebGPU's `src/core`:
 *   - `class Compute` (src/core/gpu.ts:2-67): device, budget-tracked buffers, ordered
 *     writes, dispatch, copies, clears, fences, read-back, deferred device faults;
 *   - the WGSL kernels (src/core/shaders.ts:13-181, src/core/qwen-shaders.ts:27-34),
 *     each a launcher below with the WGSL uniform parameter list;
 *   - the resident weight pager (src/core/pager.ts:7-47): weights live in HBM, one
 *     device allocation per tensor, so there is no paging slot;
 *   - the dense decoder step of `PagedEngine.forward/denseLayer` and the Gemma-3 body
 *     (src/core/engine.ts:138-180, 217-251) as `wgd_model_*`, run natively so a
 *     decode step is one captured HIP graph rather than hundreds of host calls.
 *
 * Conventions
 *   - Every function returns 0 on success and a non-zero WGD_E* status on failure.
 *     The message is kept per context and read with wgd_last_error(); the host
 *     bindings turn it into a thrown Error, as Compute does (gpu.ts:20-27).
 *   - All launches are asynchronous and strictly ordered on the context's single HIP
 *     stream, which gives the WebGPU queue-ordering guarantee (verify.ts:67-74).
 *     A device fault raised by an earlier launch is reported by the next wgd_done(),
 *     wgd_read() or model call (the deferred `fault` of gpu.ts:9,20-23).
 *   - Buffers are opaque handles owned by the context; host pointers are borrowed
 *     only for the duration of a call.
 *   - Quantization type ids are GGUF's (QUANTS, src/core/gguf.ts:6-11):
 *     F32 0, F16 1, Q4_0 2, Q8_0 8, Q4_K 12, Q5_K 13, Q6_K 14.
 *   - A context is used from one host thread at a time (engine.ts:258 `busy` guard).
 */
#ifndef WGD_H
#define WGD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WGD_OK 0
#define WGD_E_INVALID 1   /* bad argument, shape, type or size                 */
#define WGD_E_BUDGET 2    /* budget exceeded (gpu.ts:26)                       */
#define WGD_E_DEVICE 3    /* HIP runtime error or deferred device fault        */
#define WGD_E_NONFINITE 4 /* greedy sampling found no finite logit (engine.ts:308) */
#define WGD_E_STATE 5     /* call out of order (model not ready, destroyed)    */

typedef struct wgd_context wgd_context;
typedef struct wgd_buffer wgd_buffer;
typedef struct wgd_model wgd_model;

/* ---------------------------------------------------------------- runtime
 * Compute (src/core/gpu.ts:2-67). */

/* Compute constructor + init(): open HIP device `device`, create the ordered stream.
 * `budget_bytes` is the allocation ceiling (gpu.ts:7,26); 0 means the device's free
 * memory. On failure *out is NULL and the status says why (a NULL context message is
 * available from wgd_last_error(NULL)). */
int wgd_create(int32_t device, uint64_t budget_bytes, wgd_context **out);
/* Compute.dispose (gpu.ts:66): frees every buffer and model of the context. */
void wgd_destroy(wgd_context *ctx);
/* Message of the last failing call on `ctx` (thread-local message when ctx is NULL). */
const char *wgd_last_error(const wgd_context *ctx);
/* Compute.adapterName (gpu.ts:15). */
const char *wgd_adapter_name(const wgd_context *ctx);
/* Compute.allocated / Compute.peak (gpu.ts:4-5). */
uint64_t wgd_allocated(const wgd_context *ctx);
uint64_t wgd_peak(const wgd_context *ctx);

/* Compute.buffer (gpu.ts:24-30): size rounded up to 4 bytes, minimum 4; zero-filled. */
int wgd_buffer_create(wgd_context *ctx, uint64_t size, const char *label, wgd_buffer **out);
/* Compute.destroy (gpu.ts:31). */
int wgd_buffer_destroy(wgd_context *ctx, wgd_buffer *buf);
uint64_t wgd_buffer_size(const wgd_buffer *buf);
/* WeightPager.page (pager.ts:25-44) with paging collapsed: upload a whole rows x cols weight
 * matrix of GGUF `type` once, in the layout the kernels read fastest. Q4_K, Q5_K and Q6_K
 * (and Q8_0 / Q4_0 of a width that is a multiple of 64) are rearranged on the device into a
 * planar layout of the same bits (16-byte quant chunks tiled by 16 rows, block headers and
 * scales in separate planes); other types keep the GGUF bytes. Decoded values are unchanged. The buffer is accepted by wgd_matmul, wgd_matvec and
 * wgd_embed for that type and shape. `bytes` must equal rows*rowBytes. */
int wgd_upload_weights(wgd_context *ctx, int32_t type, uint32_t cols, uint32_t rows,
                       const void *data, uint64_t bytes, const char *label, wgd_buffer **out);
/* The context's HIP stream (hipStream_t), for hosts that time or order work against it. */
void *wgd_stream(const wgd_context *ctx);
/* Compute.write (gpu.ts:32): ordered host→device copy of `bytes` at `offset`. */
int wgd_write(wgd_context *ctx, wgd_buffer *buf, uint64_t offset, const void *data, uint64_t bytes);
/* Compute.read (gpu.ts:61-65): waits for all queued work, then copies back. */
int wgd_read(wgd_context *ctx, const wgd_buffer *buf, uint64_t offset, void *out, uint64_t bytes);
/* Compute.copy (gpu.ts:52-54). */
int wgd_copy(wgd_context *ctx, const wgd_buffer *src, wgd_buffer *dst, uint64_t size,
             uint64_t src_offset, uint64_t dst_offset);
/* Compute.clear (gpu.ts:55-59): zero-fill the whole buffer. */
int wgd_clear(wgd_context *ctx, wgd_buffer *buf);
/* Compute.done (gpu.ts:60): wait for queued work and surface deferred faults. */
int wgd_done(wgd_context *ctx);

/* ---------------------------------------------------------------- kernels
 * One launcher per WGSL pipeline; parameters are the WGSL uniform fields. All tensors
 * are f32 unless stated; batch-major [batch][dim] layout as in engine.ts:94-96. */

/* matmulShader(type) (shaders.ts:39-54), dispatched by `linear` (engine.ts:125-137):
 *   y[b*stride + rowBase + r] = sum_c deq(W)[r*cols + c] * x[(b+inputOffset)*cols + c]
 * for r < rows, b < batch. W holds GGUF blocks of `type` (rows x cols, row-major,
 * quantized along cols). Batch 1 runs the decode matvec (wgd_quantize + wgd_matvec) where
 * the type and layout allow it; batches above 4, and any batch on planar weights, run the
 * dequant-GEMM on bf16 MFMA with a split-precision activation operand; the rest runs a
 * generic f32 kernel. */
int wgd_matmul(wgd_context *ctx, int32_t type, const wgd_buffer *w, const wgd_buffer *x,
               wgd_buffer *y, uint32_t cols, uint32_t rows, uint32_t stride, uint32_t row_base,
               uint32_t input_offset, uint32_t batch);
/* The decode matvec split in its two steps, for hosts that drive single ops:
 * wgd_quantize turns an f32 activation row of `cols` elements into the quantized form the
 * integer matvec reads (buffer of wgd_quantized_bytes(cols)), optionally as RMSNorm(x) * w
 * (normShader, shaders.ts:55-68, with w = norm_weight, NULL for none); wgd_matvec then
 * computes y[row_base + r] = sum_c deq(W)[r][c] x[c] for weights uploaded with
 * wgd_upload_weights (every type; Q8_0 and Q4_0 in the planar layout, F16 and F32 rows of a
 * width that is a multiple of 16). wgd_matmul with batch 1 runs exactly these two. */
uint64_t wgd_quantized_bytes(uint32_t cols);
int wgd_quantize(wgd_context *ctx, const wgd_buffer *x, uint32_t cols, const wgd_buffer *norm_weight,
                 float epsilon, wgd_buffer *qx);
int wgd_matvec(wgd_context *ctx, int32_t type, const wgd_buffer *w, const wgd_buffer *qx, wgd_buffer *y,
               uint32_t cols, uint32_t rows, uint32_t row_base);
/* wgd_matvec once per launch shape that the decode step's launch-shape measurement may pick
 * for this matrix and input (the cost-model shape first; F16/F32 matrices have none): shape k
 * writes y[k * rows + r], for k < *count <= max_shapes, and y must hold max_shapes * rows
 * floats. Every shape computes the same bits, which is what a caller checks with it; no
 * reference counterpart (the measurement is this library's own). */
int wgd_matvec_shapes(wgd_context *ctx, int32_t type, const wgd_buffer *w, const wgd_buffer *qx, wgd_buffer *y,
                      uint32_t cols, uint32_t rows, uint32_t max_shapes, uint32_t *count);
/* decodeWeight (src/core/quant.ts:6-29) for `count` consecutive elements: out[i] =
 * deq(W)[i] rounded once to f32, bit-identical to the reference's decode. */
int wgd_dequant(wgd_context *ctx, int32_t type, const wgd_buffer *w, wgd_buffer *out,
                uint64_t count);
/* normShader (shaders.ts:55-68): y = x * inverseSqrt(mean(x^2) + eps) * w per row of n. */
int wgd_norm(wgd_context *ctx, const wgd_buffer *x, const wgd_buffer *w, wgd_buffer *y,
             uint32_t n, float epsilon, uint32_t batch);
/* ropeShader (shaders.ts:69-87): per (token, head) RMS-normalise with `w` (Q/K norm),
 * then half-split rotation of the first `rotary_dim` dims (0 = head_dim) by angle
 * (start+t)*scale/theta^(2i/rot); the tail is only normalised. In place on x. */
int wgd_rope_norm(wgd_context *ctx, wgd_buffer *x, const wgd_buffer *w, uint32_t heads,
                  uint32_t head_dim, uint32_t start, float theta, float scale, float epsilon,
                  uint32_t rotary_dim, uint32_t batch);
/* ropeNeoxShader (shaders.ts:139-152): half-split pairs (i, i+rot/2). */
int wgd_rope_neox(wgd_context *ctx, wgd_buffer *x, uint32_t heads, uint32_t head_dim,
                  uint32_t start, float theta, float scale, uint32_t rotary_dim, uint32_t batch);
/* ropeClassicShader (shaders.ts:155-168): adjacent pairs (2j, 2j+1). */
int wgd_rope_adjacent(wgd_context *ctx, wgd_buffer *x, uint32_t heads, uint32_t head_dim,
                      uint32_t start, float theta, float scale, uint32_t rotary_dim,
                      uint32_t batch);
/* attentionShader(context) (shaders.ts:88-122): causal GQA for query token b and head h
 * over keys t in [end - min(end, window), end), end = start + b + 1, key/value row at
 * ring slot t % capacity of a [capacity][kvHeads][hd] cache, kv head h/(heads/kvHeads).
 * capacity 0 selects `context` as in the WGSL constant. hd <= 512. Split-K over the
 * key range with an online-softmax combine. */
int wgd_attention(wgd_context *ctx, const wgd_buffer *q, const wgd_buffer *k,
                  const wgd_buffer *v, wgd_buffer *y, uint32_t heads, uint32_t kv_heads,
                  uint32_t head_dim, uint32_t start, float scale, uint32_t window,
                  uint32_t capacity, uint32_t context, uint32_t batch);
/* wgd_attention with no allocation: no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and the same results, bit for bit: the
 * split-K partials go to a static array in the library's device memory (one per GPU, held
 * until the process ends) instead of context scratch. Sizes whose partials exceed
 * wgd_attention_noalloc_limit() floats fail with WGD_E_INVALID. Calls on one GPU share the
 * array: calls that overlap on one GPU (two streams) race. */
int wgd_attention_noalloc(wgd_context *ctx, const wgd_buffer *q, const wgd_buffer *k,
                          const wgd_buffer *v, wgd_buffer *y, uint32_t heads, uint32_t kv_heads,
                          uint32_t head_dim, uint32_t start, float scale, uint32_t window,
                          uint32_t capacity, uint32_t context, uint32_t batch);
/* wgd_attention over an f16 K/V ring: the same arguments and semantics, with k and v
 * holding [capacity][kvHeads][hd] IEEE halves (2 bytes per element) instead of f32. Scores,
 * softmax and the weighted sum run in f32 on the exactly widened values. The reference
 * allocates its rings at 4 bytes per element (engine.ts:98-101, sized by attentionMemory,
 * context.ts:16-24); the f16 ring halves that memory and the bytes each decode step reads. */
int wgd_attention_f16kv(wgd_context *ctx, const wgd_buffer *q, const wgd_buffer *k,
                        const wgd_buffer *v, wgd_buffer *y, uint32_t heads, uint32_t kv_heads,
                        uint32_t head_dim, uint32_t start, float scale, uint32_t window,
                        uint32_t capacity, uint32_t context, uint32_t batch);
/* cacheKV's ring copy (engine.ts:120-124, Compute.copy of cacheCopies' ranges) into an f16
 * ring: dst[dst_offset + i] = f16(src[src_offset + i]) for i < count, rounded to nearest
 * (ties to even). Offsets and count are in elements (floats of src, halves of dst). */
int wgd_kv_store_f16(wgd_context *ctx, const wgd_buffer *src, wgd_buffer *dst, uint64_t count,
                     uint64_t src_offset, uint64_t dst_offset);
/* Floats of the static scratch of wgd_attention_noalloc (8 Mi floats, 32 MiB). */
uint64_t wgd_attention_noalloc_limit(void);
/* addShader (shaders.ts:123-128): state += delta. */
int wgd_add(wgd_context *ctx, const wgd_buffer *delta, wgd_buffer *state, uint32_t n);
/* siluShader (qwen-shaders.ts:27-34): y = g / (1 + exp(-g)) * up. */
int wgd_silu(wgd_context *ctx, const wgd_buffer *gate, const wgd_buffer *up, wgd_buffer *y,
             uint32_t n);
/* geluShader (shaders.ts:129-137): y = 0.5 g (1 + tanh(0.7978845608 (g + 0.044715 g^3))) up. */
int wgd_gelu(wgd_context *ctx, const wgd_buffer *gate, const wgd_buffer *up, wgd_buffer *y,
             uint32_t n);
/* biasAddShader (shaders.ts:170-175): y[i] += b[i % width]. */
int wgd_bias_add(wgd_context *ctx, wgd_buffer *y, const wgd_buffer *b, uint32_t n,
                 uint32_t width);
/* activateShader (shaders.ts:177-181): in-place x = x / (1 + exp(-x)). */
int wgd_activate(wgd_context *ctx, wgd_buffer *x, uint32_t n);
/* sample(T=0) (engine.ts:305-309) on the device: index of the first strict maximum over
 * the finite entries of logits[0..n). Writes an int32 to out (-1 when none is finite)
 * and, when host_index is non-NULL, waits and returns it there, failing with
 * WGD_E_NONFINITE when no entry is finite. */
int wgd_argmax(wgd_context *ctx, const wgd_buffer *logits, uint32_t n, wgd_buffer *out,
               int32_t *host_index);
/* sample (engine.ts:305-324) on the device for logits[0..n): the first finite maximum
 * when temperature is 0, else the top_k finite logits (ties to the lower index),
 * exp((l - best) / T) in f64, the top_p prefix and a draw with the index-th output of
 * splitmix64(seed) as Math.random(). Waits; returns the token (WGD_E_NONFINITE when no
 * logit is finite, WGD_E_INVALID for settings the reference rejects). */
int wgd_sample(wgd_context *ctx, const wgd_buffer *logits, uint32_t n, double temperature, uint32_t top_k,
               double top_p, uint64_t seed, uint32_t index, int32_t *token);
/* Embedding gather of `forward` (engine.ts:140-145) on the device:
 * out[b*hidden + i] = f32(deq(table)[ids[b]*hidden + i] * scale) with the product taken
 * in f64 (scale = sqrt(hidden) for Gemma 3, else 1). ids is int32[n]. */
int wgd_embed(wgd_context *ctx, int32_t type, const wgd_buffer *table, const wgd_buffer *ids,
              wgd_buffer *out, uint32_t hidden, uint32_t n, double scale);

/* ---------------------------------------------------------------- measurement
 * No reference counterpart: `launches` back-to-back plain streaming reads of `bytes`
 * (multiple of 16), launch i reading copy i % copies of src (copies laid out `bytes`
 * rounded up to 4 KiB apart), by `workgroups` workgroups of `threads` threads with `depth`
 * (4, 8, 16) 16-byte loads in flight per lane, a contiguous range per workgroup. With
 * out_floats > 0 each workgroup also stores its share of an out_floats-long result into
 * out. It is the per-launch floor of a kernel that reads those bytes once (bench.py
 * --probe); the loop runs in the library so the host does not pace short launches. */
int wgd_probe_read(wgd_context *ctx, const wgd_buffer *src, uint64_t bytes, uint32_t copies,
                   uint32_t launches, uint32_t workgroups, uint32_t threads, uint32_t depth,
                   wgd_buffer *out, uint32_t out_floats);

/* ---------------------------------------------------------------- model
 * The dense decoder step (engine.ts:138-180, 217-251) with resident weights. */

typedef struct wgd_model_config {
  int32_t family;         /* 0 dense decoder (llama/qwen2/qwen3), 1 gemma3  (gguf.ts:141)   */
  int32_t rope_adjacent;  /* 1 = adjacent pairs ('norm', arch llama), 0 = half-split (:168) */
  int32_t hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
  int32_t rotary_dim;     /* rotated dims per head (gguf.ts:166)                          */
  int32_t window;         /* attention window for local/sliding layers; 0 = context        */
  int32_t period;         /* gemma3: layer l is global iff l % period == period-1 (:162)   */
  int32_t qk_norm, ffn_gate, gelu;             /* detected from tensors (gguf.ts:197-199) */
  int32_t bias_q, bias_k, bias_v, bias_output;
  int32_t tied_output;    /* no output.weight: the head reuses token_embd (engine.ts:178) */
  int32_t context;        /* LoadOptions.contextLength (engine.ts:55)                      */
  int32_t batch;          /* LoadOptions.batchSize: largest forward() chunk                 */
  float epsilon, theta, local_theta, attention_scale, rope_scale;
  double embed_scale;     /* sqrt(hidden) for gemma3, 1 otherwise (engine.ts:143)          */
  int32_t kv_f16;         /* K/V rings in f16 (1) or f32 as the reference (0, engine.ts:98-101);
                             f16 rings store values rounded to nearest even, math stays f32 */
} wgd_model_config;

/* Allocate work buffers and per-layer K/V rings (capacities[l] slots each, from
 * attentionMemory, context.ts:16-24; 4 bytes per element, 2 with kv_f16). */
int wgd_model_create(wgd_context *ctx, const wgd_model_config *cfg, const int32_t *capacities,
                     wgd_model **out);
/* Upload one GGUF tensor (raw block bytes as stored in the file, `bytes` long).
 * 1-D tensors (norm vectors, biases) are decoded to f32 on the device as in
 * engine.ts:102-109. Names are GGUF's ("blk.3.attn_q.weight", ...). */
int wgd_model_tensor(wgd_model *m, const char *name, int32_t type, int32_t n_dims,
                     const uint64_t *dims, const void *data, uint64_t bytes);
/* Check that every tensor the config needs is present and shaped as modelConfig
 * validates it (gguf.ts:188-241); after this the model accepts forward calls. */
int wgd_model_ready(wgd_model *m);
/* PagedEngine.forward (engine.ts:138-180) for ids[0..n) at positions start..start+n-1
 * (n <= batch). When logits or argmax is non-NULL the last row's logits are produced
 * (vocab f32 copied to `logits`; the next token to `argmax`, WGD_E_NONFINITE if no logit
 * is finite: the greedy id, or with sampling set the draw for position start + n). */
int wgd_model_forward(wgd_model *m, const int32_t *ids, int32_t n, int32_t start,
                      float *logits, int32_t *argmax);
/* The decode loop of generate (engine.ts:290-298) kept on the device: for i < count, run
 * forward([token_i], start+i) and take token_{i+1} by the model's token pick (greedy, or
 * sampled as set by wgd_model_sampling); token_0 = `token`. Writes token_1..token_count to
 * out_tokens. Each step is one replay of a captured HIP graph (one per pick mode);
 * positions and ids never leave the device between steps. */
int wgd_model_decode(wgd_model *m, int32_t token, int32_t start, int32_t count,
                     int32_t *out_tokens);
/* The token pick of generate (engine.ts:261-264, 292, 305-324) for wgd_model_forward and
 * wgd_model_decode: temperature 0 is greedy; otherwise top_k / top_p sampling on the
 * device, where Math.random() becomes the p-th output of splitmix64(seed) for the token
 * at position p (the same tokens whether decoded eagerly, in chunks or by graph replay).
 * Validated as the reference validates GenerationOptions (WGD_E_INVALID). */
int wgd_model_sampling(wgd_model *m, double temperature, uint32_t top_k, double top_p, uint64_t seed);
void wgd_model_destroy(wgd_model *m);
/* Measurement, no reference counterpart: the mean device time in microseconds (HIP events
 * on the context's stream) of `reps` back-to-back launches of the decode step's attention
 * of `layer` at position `pos` (Q/K norm and RoPE of the token, its K/V written to ring slot
 * pos % capacity, split-K attention over the keys before it, merge and quantization for the
 * O projection), on the token's current q/k/v work buffers. It overwrites that ring slot, so
 * call it where the slot holds no live key. Models whose decode step has no fused attention
 * launch return WGD_E_INVALID. */
int wgd_model_attention_timing(wgd_model *m, int32_t layer, int32_t pos, int32_t reps, double *us);

#ifdef __cplusplus
}
#endif
#endif /* WGD_H */
