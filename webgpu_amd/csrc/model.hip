// model.hip — the dense decoder step of PagedEngine (src/core/engine.ts:138-180, denseLayer
// :217-251, Gemma-3 body :158-174) with every weight resident in HBM.
//
// Two execution paths share the kernels:
//   * forward(n > 1): the prompt chunk, batch-major [n][dim] buffers as in engine.ts:94-96,
//     batched dequant-GEMM on MFMA, KV ring append, split-K attention;
//   * the decode step (n = 1): RMSNorm folded into the consuming matvec, SwiGLU/GeGLU
//     folded into a paired gate/up matvec, residual adds folded into the O and down
//     projections, the greedy argmax and token hand-off on the device. Position and token
//     id live in device memory, so the step is captured once as a HIP graph and replayed
//     for every generated token without host round-trips (the reference fences after every
//     layer, engine.ts:152-174, and reads logits back for a CPU argmax, :179, :291).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <utility>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "internal.h"
#include "decode.h"
#include "attention.h"
#include "matvec.h"
#include "model.h"

using namespace wgd;

namespace {

struct Layer {
  Matrix q, k, v, o, gate, up, down;
  float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  float *post_attn = nullptr, *post_ffw = nullptr;
  float *bq = nullptr, *bk = nullptr, *bv = nullptr, *bo = nullptr;
  void *kc = nullptr, *vc = nullptr;  // K/V rings: f32, or f16 with kv_f16
  uint32_t cap = 0;
};


enum Slot { S_ATTN_NORM, S_Q, S_K, S_V, S_O, S_QB, S_KB, S_VB, S_OB, S_QN, S_KN, S_POST_ATTN, S_FFN_NORM,
            S_GATE, S_UP, S_DOWN, S_POST_FFW, S_COUNT };
const char *kSlotNames[S_COUNT] = {"attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
                                   "attn_output.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias",
                                   "attn_output.bias", "attn_q_norm.weight", "attn_k_norm.weight",
                                   "post_attention_norm.weight", "ffn_norm.weight", "ffn_gate.weight",
                                   "ffn_up.weight", "ffn_down.weight", "post_ffw_norm.weight"};

}  // namespace

struct wgd_model {
  wgd_context *ctx = nullptr;
  wgd_model_config c{};
  std::vector<Layer> L;
  std::vector<uint32_t> seen;   // bitmask of uploaded slots per layer
  Matrix embd, output;
  float *out_norm = nullptr;
  bool have_embd = false, have_output = false, ready = false;
  // work buffers, [batch][dim]
  float *hidden = nullptr, *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr,
        *proj = nullptr, *gate = nullptr, *up = nullptr, *prod = nullptr, *down = nullptr, *logits = nullptr;
  int32_t *ids = nullptr;
  StepState *state = nullptr;
  int32_t *tokens = nullptr;    // decode output ring, one per position
  int32_t *argmax_buf = nullptr;
  uint64_t *arg_part = nullptr; uint32_t arg_entries = 0;  // head argmax keys (quantized path)
  float *att_part = nullptr; uint64_t att_part_floats = 0;
  float *res_sq = nullptr;        // per-token segment sums of squares of a deferred prompt RMSNorm
  GemmScratch gemm_part;          // split-K partial sums of the prompt GEMMs
  // Quantized-activation decode path (every matrix Q4_K, Q6_K or Q8_0): activation buffers
  // in the QX format.
  bool qpath = false;
  bool fused_attention = false;  // decode attention in one pass (head dims 64 / 128 / 256)
  // RoPE inverse frequencies of the decode attention: [0] the model's theta, [1] Gemma's local
  double *inv_freq[2] = {nullptr, nullptr};
  float *rope_cs[2] = {nullptr, nullptr};  // this token's rotation tables (token_start)
  float2 *rope_batch[2] = {nullptr, nullptr};  // a prompt batch's rotations (rope_table)
  void *qx_attn = nullptr, *qx_ffn = nullptr, *qx_o = nullptr, *qx_down = nullptr, *qx_head = nullptr;
  hipGraph_t graph = nullptr;
  // the sampling variant of the decode step (its own graph); settings in device memory
  bool sampling = false;
  SampleParams *sample_params = nullptr;
  void *sample_scratch = nullptr;
  hipGraph_t graph_s = nullptr;
  hipGraphExec_t exec_s = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<void *> owned;
};

namespace {

int alloc(wgd_model *m, uint64_t bytes, const char *label, void **out) {
  int rc = ctx_alloc(m->ctx, bytes, label, out);
  if (rc == WGD_OK) m->owned.push_back(*out);
  return rc;
}
template <class T> int alloc_t(wgd_model *m, uint64_t count, const char *label, T **out) {
  void *p = nullptr;
  int rc = alloc(m, count * sizeof(T), label, &p);
  *out = (T *)p;
  return rc;
}

bool is_gemma(const wgd_model *m) { return m->c.family == 1; }
bool local_layer(const wgd_model *m, int l) { return m->c.period > 1 && l % m->c.period != m->c.period - 1; }

uint32_t window_of(const wgd_model *m, int l) {
  if (is_gemma(m)) return local_layer(m, l) ? (uint32_t)m->c.window : (uint32_t)m->c.context;
  return m->c.window > 0 ? (uint32_t)m->c.window : (uint32_t)m->c.context;
}

hipError_t bias(hipStream_t s, float *y, const float *b, uint32_t n, uint32_t width) {
  return b ? bias_add(s, y, b, n * width, width) : hipSuccess;
}

// The RoPE of layer l: theta, scale, mode (0 Q/K norm + half-split, 1 half-split,
// 2 adjacent), rotary width (0 = head dim) and norm epsilon.
struct RopeParams { float theta, scale, eps; uint32_t rot; int mode; };
static RopeParams rope_params(wgd_model *m, int l) {
  const wgd_model_config &c = m->c;
  if (is_gemma(m)) {
    const bool loc = local_layer(m, l);
    return RopeParams{loc ? c.local_theta : c.theta, loc ? 1.f : c.rope_scale, c.epsilon, 0, 0};
  }
  if (c.qk_norm) return RopeParams{c.theta, c.rope_scale, c.epsilon, (uint32_t)c.rotary_dim, 0};
  return RopeParams{c.theta, c.rope_scale, 0.f, (uint32_t)c.rotary_dim, c.rope_adjacent ? 2 : 1};
}

// Attention of one layer, with RoPE and the KV append unless `prepared` (the Q/K/V GEMM
// finish did them); positions from start (host) or start_dev.
hipError_t attention_block(wgd_model *m, int l, uint32_t n, uint32_t start, const int32_t *start_dev,
                           bool prepared = false, uint16_t *xs = nullptr, bool *xs_written = nullptr) {
  const wgd_model_config &c = m->c;
  Layer &L = m->L[l];
  hipStream_t s = m->ctx->stream;
  const uint32_t hd = c.head_dim, kd = c.kv_heads * hd;
  if (!prepared) {
    const RopeParams r = rope_params(m, l);
    const float *qn = r.mode == 0 ? L.q_norm : nullptr, *kn = r.mode == 0 ? L.k_norm : nullptr;
    WGD_HIP(rope(s, m->q, qn, c.heads, hd, start, start_dev, r.theta, r.scale, r.eps, r.rot, n, r.mode));
    WGD_HIP(rope(s, m->k, kn, c.kv_heads, hd, start, start_dev, r.theta, r.scale, r.eps, r.rot, n, r.mode));
    WGD_HIP(kv_append(s, m->k, m->v, L.kc, L.vc, kd, n, start, start_dev, L.cap, c.kv_f16 != 0));
  }
  AttnArgs a;
  a.q = m->q; a.k = L.kc; a.v = L.vc; a.y = m->att; a.kv16 = c.kv_f16 != 0;
  a.heads = c.heads; a.kv_heads = c.kv_heads; a.hd = hd; a.start = start; a.start_dev = start_dev;
  a.scale = c.attention_scale; a.window = window_of(m, l); a.capacity = L.cap; a.batch = n;
  a.partial = m->att_part; a.partial_floats = (uint32_t)m->att_part_floats;
  a.xs = xs; a.xs_written = xs_written;
  return attention(s, a);
}

// The decode token's attention in one fused pass (Q/K norm, RoPE, KV append, attention,
// merge), writing m->att and its quantized form for the O projection.
hipError_t decode_attention_layer(wgd_model *m, int l, const QXOut &qx) {
  const wgd_model_config &c = m->c;
  Layer &L = m->L[l];
  DecodeAttnArgs a;
  a.q = m->q; a.k = m->k; a.v = m->v; a.kc = L.kc; a.vc = L.vc; a.kv16 = c.kv_f16 != 0;
  a.q_norm = nullptr; a.k_norm = nullptr;
  a.partial = m->att_part; a.y = m->att; a.qx = qx; a.pos = &m->state->pos;
  a.heads = c.heads; a.kv_heads = c.kv_heads; a.hd = c.head_dim; a.capacity = L.cap; a.window = window_of(m, l);
  a.scale = c.attention_scale; a.eps = c.epsilon;
  a.rope = m->rope_cs[0];
  if (is_gemma(m)) {
    a.mode = 0; a.rot = 0; a.q_norm = L.q_norm; a.k_norm = L.k_norm;
    if (local_layer(m, l)) a.rope = m->rope_cs[1];
  } else if (c.qk_norm) {
    a.mode = 0; a.rot = c.rotary_dim; a.q_norm = L.q_norm; a.k_norm = L.k_norm;
  } else {
    a.mode = c.rope_adjacent ? 2 : 1; a.rot = c.rotary_dim;
  }
  return decode_attention(m->ctx->stream, a);
}

// The prompt GEMM groups of a layer: Q, K and V of the normed input in one launch, and gate
// with up finishing in the GLU (prod and its split for the down GEMM).
static GemmGroup qkv_group(wgd_model *m, const Layer &L) {
  const wgd_model_config &c = m->c;
  const uint32_t qd = c.heads * c.head_dim, kd = c.kv_heads * c.head_dim;
  GemmGroup g;
  g.job[0] = GemmJob{&L.q, m->q, qd, 0};
  g.job[1] = GemmJob{&L.k, m->k, kd, 0};
  g.job[2] = GemmJob{&L.v, m->v, kd, 0};
  g.n = 3; g.keep_partials = true;
  return g;
}
static GemmGroup glu_group(wgd_model *m, const Layer &L) {
  const uint32_t F = m->c.intermediate;
  GemmGroup g;
  g.job[0] = GemmJob{&L.gate, m->gate, F, 0};
  g.job[1] = GemmJob{&L.up, m->up, F, 0};
  g.n = 2; g.glu_out = m->prod; g.glu_act = m->c.gelu;
  return g;
}

// A residual projection kept as split-K partials for the fused norm finish.
static GemmGroup res_group(wgd_model *m, const Matrix &W) {
  GemmGroup g;
  g.job[0] = GemmJob{&W, m->hidden, (uint32_t)m->c.hidden, 0};
  g.n = 1; g.keep_partials = true;
  return g;
}

// n tokens already gathered into m->hidden (a prompt chunk, or one decode token on the
// generic path with its position in device memory).
hipError_t layers_batched(wgd_model *m, uint32_t n, uint32_t start, const int32_t *start_dev = nullptr) {
  const wgd_model_config &c = m->c;
  hipStream_t s = m->ctx->stream;
  const uint32_t H = c.hidden, qd = c.heads * c.head_dim, kd = c.kv_heads * c.head_dim, F = c.intermediate;
  // The GEMMs of one input (q, k, v; gate, up) share its bf16 split (xs_of names the buffer
  // it was made from and is cleared whenever that buffer is rewritten). RMSNorm and the GLU
  // write the split themselves when the GEMM after them runs on it; the O and down GEMMs
  // then add straight into the residual stream.
  GemmScratch gs = m->gemm_part;
  auto norm_for = [&](const float *w, const Matrix &first) -> hipError_t {
    if (!gemm_splits_input(first, &gs, n)) {
      gs.xs_of = nullptr;
      return norm(s, m->hidden, w, m->normed, H, c.epsilon, n);
    }
    gs.xs_of = m->normed; gs.xs_cols = H; gs.xs_batch = n;
    return norm_split(s, m->hidden, w, m->normed, gs.xs, H, c.epsilon, n);
  };
  const bool gemma = is_gemma(m);
  // the batch's RoPE rotations, once for every layer (Gemma: global and local theta)
  if (m->rope_batch[0]) {
    int lg = 0, ll = 0;  // a global and a local layer (Gemma)
    while (lg + 1 < c.layers && local_layer(m, lg)) lg++;
    while (ll + 1 < c.layers && !local_layer(m, ll)) ll++;
    const RopeParams r0 = rope_params(m, lg);
    WGD_HIP(rope_table(s, m->rope_batch[0], r0.rot ? r0.rot : c.head_dim, n, start, start_dev, r0.theta, r0.scale));
    if (gemma && m->rope_batch[1]) {
      const RopeParams r1 = rope_params(m, ll);
      WGD_HIP(rope_table(s, m->rope_batch[1], c.head_dim, n, start, start_dev, r1.theta, r1.scale));
    }
  }
  // The input norm of the next GEMM group is deferred into that group's finish (DeferredNorm)
  // while dn.sq is set: the split in gs.xs then holds x * w, not the normed x.
  DeferredNorm dn;
  // A residual projection (O, down) into m->hidden: with the next RMSNorm fused into its
  // split-K finish when that norm feeds a split-input GEMM (then returns true: the split of
  // m->normed is ready), else added by the GEMM's own reduction, else the generic path. When
  // the GEMM group after the norm has its own finish (`deferred`: the grouped Q/K/V or
  // gate/up), the norm factor is left to that finish, so the residual finish needs no
  // row-wide sum and spreads over every CU; otherwise one workgroup per token forms the norm
  // and writes m->normed as well.
  auto residual = [&](const Matrix &W, const float *x, const float *bias_w, const float *post_w,
                      const float *next_w, const Matrix *next_first, bool deferred) -> std::pair<hipError_t, bool> {
    if (!bias_w && gemm_splits_input(W, &gs, n)) {
      // Gemma's post-norm needs the whole row, so its finish is the per-token one
      if (next_w && next_first && gemm_splits_input(*next_first, &gs, n) && (gemma ? H <= 16384 : deferred || H <= 16384)) {
        GemmGroup g = res_group(m, W);
        uint32_t splits = 0;
        g.splits = &splits;
        hipError_t e = gemm_group(s, g, x, n, &gs);
        if (e == hipSuccess && deferred && !gemma) {
          e = residual_split(s, gs.p, splits, m->hidden, next_w, gs.xs, m->res_sq, H, n);
          dn = DeferredNorm{m->res_sq, residual_split_segs(H), H, c.epsilon};
        } else if (e == hipSuccess) {
          e = reduce_norm_split(s, gs.p, splits, m->hidden, next_w, m->normed, gs.xs, H, c.epsilon, n,
                                gemma ? post_w : nullptr);
        }
        gs.xs_of = m->normed; gs.xs_cols = H; gs.xs_batch = n;
        return {e, true};
      }
      if (!gemma) return {matmul(s, W, x, m->hidden, H, 0, 0, n, &gs, true), false};
    }
    hipError_t e = matmul(s, W, x, m->proj, H, 0, 0, n, &gs);
    if (e == hipSuccess) e = bias(s, m->proj, bias_w, n, H);
    if (e == hipSuccess) e = gemma ? norm_add(s, m->proj, post_w, m->hidden, H, c.epsilon, n) : add(s, m->proj, m->hidden, n * H);
    return {e, false};
  };
  // whether a layer's Q/K/V, and its gate/up, run as one grouped GEMM with its own finish
  auto qkv_fused = [&](const Layer &L) {
    return m->rope_batch[0] && gemm_splits_input(L.q, &gs, n) && gemm_group_ok(qkv_group(m, L), n);
  };
  auto glu_fused = [&](const Layer &L) {
    return c.ffn_gate && gemm_splits_input(L.up, &gs, n) && gemm_group_ok(glu_group(m, L), n);
  };
  bool normed_ready = false;  // the split of this layer's attention-norm input is ready (dn: deferred)
  for (int l = 0; l < c.layers; l++) {
    Layer &L = m->L[l];
    if (!normed_ready) {
      WGD_HIP(norm_for(L.attn_norm, L.q));
      dn = DeferredNorm{};
    }
    normed_ready = false;
    GemmGroup qkv = qkv_group(m, L);
    uint32_t splits = 0;
    qkv.keep_partials = true; qkv.splits = &splits;
    if (qkv_fused(L)) {
      // Q/K/V partial sums finished in one pass: bias, RoPE, K/V into the ring
      WGD_HIP(gemm_group(s, qkv, m->normed, n, &gs));
      const RopeParams r = rope_params(m, l);
      QKVFinish f;
      f.part = gs.p; f.splits = splits; f.rows_total = qd + 2 * kd; f.batch = n;
      f.bq = L.bq; f.bk = L.bk; f.bv = L.bv;
      f.qn = r.mode == 0 ? L.q_norm : nullptr; f.kn = r.mode == 0 ? L.k_norm : nullptr;
      f.q = m->q; f.kc = L.kc; f.vc = L.vc; f.capacity = L.cap; f.kv16 = c.kv_f16 != 0;
      f.heads = c.heads; f.kvh = c.kv_heads; f.hd = c.head_dim; f.rot = r.rot ? r.rot : c.head_dim;
      f.start = start; f.start_dev = start_dev;
      f.eps = r.eps; f.mode = r.mode;
      f.cs = m->rope_batch[gemma && local_layer(m, l) ? 1 : 0];
      f.xnorm = dn;
      WGD_HIP(qkv_finish(s, f));
      dn = DeferredNorm{};
      // the attention output's split for the O GEMM comes from the key-split merge
      bool written = false;
      const bool want = gemm_splits_input(L.o, &gs, n);
      WGD_HIP(attention_block(m, l, n, start, start_dev, true, want ? gs.xs : nullptr, &written));
      gs.xs_of = written ? m->att : nullptr; gs.xs_cols = qd; gs.xs_batch = n;
    } else {
      WGD_HIP(matmul(s, L.q, m->normed, m->q, qd, 0, 0, n, &gs));
      WGD_HIP(matmul(s, L.k, m->normed, m->k, kd, 0, 0, n, &gs));
      WGD_HIP(matmul(s, L.v, m->normed, m->v, kd, 0, 0, n, &gs));
      WGD_HIP(bias(s, m->q, L.bq, n, qd));
      WGD_HIP(bias(s, m->k, L.bk, n, kd));
      WGD_HIP(bias(s, m->v, L.bv, n, kd));
      WGD_HIP(attention_block(m, l, n, start, start_dev));
      gs.xs_of = nullptr;
    }
    auto ro = residual(L.o, m->att, L.bo, L.post_attn, L.ffn_norm, &L.up, glu_fused(L));
    WGD_HIP(ro.first);
    if (!ro.second) {
      WGD_HIP(norm_for(L.ffn_norm, L.up));
      dn = DeferredNorm{};
    }
    float *ffn_in = m->up;
    GemmGroup gu = glu_group(m, L);
    if (glu_fused(L)) {
      // prod in f32 only when the down projection cannot read its split
      gu.glu_f32 = !gemm_splits_input(L.down, &gs, n);
      gu.glu_norm = dn;
      dn = DeferredNorm{};
      WGD_HIP(gemm_group(s, gu, m->normed, n, &gs));  // leaves the split of prod in gs.xs
      ffn_in = m->prod;
    } else if (c.ffn_gate) {
      WGD_HIP(matmul(s, L.up, m->normed, m->up, F, 0, 0, n, &gs));
      WGD_HIP(matmul(s, L.gate, m->normed, m->gate, F, 0, 0, n, &gs));
      if (gemm_splits_input(L.down, &gs, n)) {
        WGD_HIP(glu_split(s, m->gate, m->up, m->prod, gs.xs, F, n, c.gelu));
        gs.xs_of = m->prod; gs.xs_cols = F; gs.xs_batch = n;
      } else {
        WGD_HIP(glu(s, m->gate, m->up, m->prod, n * F, c.gelu));
        gs.xs_of = nullptr;
      }
      ffn_in = m->prod;
    } else {
      WGD_HIP(matmul(s, L.up, m->normed, m->up, F, 0, 0, n, &gs));
      WGD_HIP(activate(s, m->up, n * F));
      gs.xs_of = nullptr;
    }
    const bool last = l + 1 == c.layers;
    auto rd = residual(L.down, ffn_in, nullptr, L.post_ffw, last ? nullptr : m->L[l + 1].attn_norm,
                       last ? nullptr : &m->L[l + 1].q, !last && qkv_fused(m->L[l + 1]));
    WGD_HIP(rd.first);
    normed_ready = rd.second;
  }
  return hipSuccess;
}

// Logits of row `row` of m->hidden (output norm, head matvec, greedy argmax) for the
// batched and generic paths.
hipError_t head(wgd_model *m, uint32_t row) {
  const wgd_model_config &c = m->c;
  hipStream_t s = m->ctx->stream;
  const Matrix &W = m->have_output && !c.tied_output ? m->output : m->embd;
  if (m->qpath && m->qx_head) {
    // the decode head: the row quantized with the output norm pending, then the integer matvec
    const QXOut q = qx_view(m->qx_head, c.hidden);
    WGD_HIP(quantize(s, m->hidden + (uint64_t)row * c.hidden, c.hidden, m->out_norm, q));
    WGD_HIP(mv(s, W, nullptr, qx_const(q, c.hidden, true, c.epsilon), m->logits, MV_STORE));
  } else {
    WGD_HIP(norm(s, m->hidden + (uint64_t)row * c.hidden, m->out_norm, m->normed, c.hidden, c.epsilon, 1));
    WGD_HIP(matmul(s, W, m->normed, m->logits, c.vocab, 0, 0, 1));
  }
  return argmax(s, m->logits, c.vocab, m->argmax_buf);
}

// Records state->token = argmax, tokens[step] = token, advances pos/step. A missing
// finite logit sets the error flag and feeds token 0 so later gathers stay in range.
__global__ void k_advance(StepState *st, const int32_t *arg, int32_t *tokens, uint32_t cap) {
  int32_t t = *arg;
  if (t < 0) { st->error = 1; t = 0; }
  if ((uint32_t)st->step < cap) tokens[st->step] = t;
  st->token = t;
  st->pos += 1;
  st->step += 1;
}

// The greedy pick from the head matvec's per-wavefront argmax keys (first index of the
// finite maximum; -1 when no logit is finite), then, with `advance`, the k_advance update.
__global__ __launch_bounds__(256) void k_argmax_advance(const uint64_t *part, uint32_t np, int32_t *out, StepState *st,
                                                        int32_t *tokens, uint32_t cap, int advance) {
  __shared__ uint64_t red[4];
  uint64_t k = 0;
  for (uint32_t i = threadIdx.x; i < np; i += 256) k = key_max(k, part[i]);
  k = wave_max_key(k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x != 0) return;
  const uint64_t mk = key_max(key_max(red[0], red[1]), key_max(red[2], red[3]));
  int32_t t = mk ? (int32_t)(0xFFFFFFFFu - (uint32_t)mk) : -1;
  *out = t;
  if (!advance) return;
  if (t < 0) { st->error = 1; t = 0; }
  if ((uint32_t)st->step < cap) tokens[st->step] = t;
  st->token = t;
  st->pos += 1;
  st->step += 1;
}

QXView qv(void *p, uint32_t K, bool normed = false, float eps = 0.f) { return qx_const(qx_view(p, K), K, normed, eps); }

// Matvecs of several matrices that read the same activation: one launch per group of at
// most two types that mix (Q6_K with Q4_K or Q5_K), else one per weight type.
std::vector<std::vector<MVTarget>> mv_groups(const MVTarget *t, uint32_t n) {
  std::vector<std::vector<MVTarget>> out;
  bool done[MV_MAX_SEGS] = {};
  for (uint32_t i = 0; i < n; i++) {
    if (done[i]) continue;
    std::vector<MVTarget> grp;
    const int a = t[i].w->type;
    int b = a;
    for (uint32_t j = i; j < n; j++) {
      const int ty = t[j].w->type;
      if (done[j]) continue;
      if (ty != a && b == a && mv_mixable(a, ty)) b = ty;
      if (ty == a || ty == b) { grp.push_back(t[j]); done[j] = true; }
    }
    // the heavier Q6_K segments first: their workgroups dispatch first
    std::stable_partition(grp.begin(), grp.end(), [](const MVTarget &t) { return t.w->type == Q6_K; });
    out.push_back(grp);
  }
  return out;
}
hipError_t mv_group(hipStream_t s, const MVTarget *t, uint32_t n, const QXView &x) {
  for (const auto &grp : mv_groups(t, n)) WGD_HIP(mv(s, grp.data(), (uint32_t)grp.size(), x, MV_STORE));
  return hipSuccess;
}

// The decode step's matvec launch shapes, measured on this model's weights before any state
// lives in the buffers the launches write (mv_tune: every candidate computes the same bits).
// The launches are the ones decode_step_q makes, grouped by weight-type signature, each
// timed over the layers that share it.
hipError_t tune_decode(wgd_model *m) {
  const wgd_model_config &c = m->c;
  hipStream_t s = m->ctx->stream;
  const uint32_t H = c.hidden, qd = c.heads * c.head_dim, F = c.intermediate;
  const bool gemma = is_gemma(m);
  typedef std::vector<int> Sig;
  auto sig_of = [](const std::vector<MVTarget> &g) {
    Sig k;
    for (const MVTarget &t : g) { k.push_back(t.w->type); k.push_back((int)t.w->rows); k.push_back(t.w1 ? 1 : 0); }
    return k;
  };
  // Q, K and V of the normed input
  {
    std::map<Sig, std::vector<MVTarget>> sets;
    std::map<Sig, uint32_t> width;
    for (int l = 0; l < c.layers; l++) {
      const Layer &L = m->L[l];
      MVTarget qkv[3];
      qkv[0].w = &L.q; qkv[0].y = m->q; qkv[0].bias = L.bq;
      qkv[1].w = &L.k; qkv[1].y = m->k; qkv[1].bias = L.bk;
      qkv[2].w = &L.v; qkv[2].y = m->v; qkv[2].bias = L.bv;
      for (const auto &g : mv_groups(qkv, 3)) {
        const Sig k = sig_of(g);
        sets[k].insert(sets[k].end(), g.begin(), g.end());
        width[k] = (uint32_t)g.size();
      }
    }
    for (const auto &kv : sets)
      WGD_HIP(mv_tune(s, kv.second.data(), (uint32_t)(kv.second.size() / width[kv.first]), width[kv.first],
                      qv(m->qx_attn, H, true, c.epsilon), MV_STORE));
  }
  // O (into the residual, re-quantized with ffn_norm; Gemma: stored for the post-norm), the
  // gated gate/up pair, and down
  MVOut to_ffn;
  to_ffn.q = qx_view(m->qx_ffn, H); to_ffn.norm_w = m->L[0].ffn_norm;
  MVOut to_down;
  to_down.q = qx_view(m->qx_down, F);
  MVOut next;
  next.q = qx_view(m->qx_attn, H); next.norm_w = m->L[0].attn_norm;
  std::map<Sig, std::vector<MVTarget>> o_sets, gu_sets, dn_sets;
  for (int l = 0; l < c.layers; l++) {
    const Layer &L = m->L[l];
    MVTarget o;
    o.w = &L.o; o.bias = L.bo; o.y = gemma ? m->proj : m->hidden;
    o_sets[sig_of({o})].push_back(o);
    if (c.ffn_gate) {
      MVTarget gu;
      gu.w = &L.gate; gu.w1 = &L.up; gu.y = m->prod;
      gu_sets[sig_of({gu})].push_back(gu);
    }
    MVTarget dn;
    dn.w = &L.down; dn.y = gemma ? m->down : m->hidden;
    dn_sets[sig_of({dn})].push_back(dn);
  }
  for (const auto &kv : o_sets)
    WGD_HIP(mv_tune(s, kv.second.data(), (uint32_t)kv.second.size(), 1, qv(m->qx_o, qd), gemma ? MV_STORE : MV_ADD,
                    gemma ? nullptr : &to_ffn));
  for (const auto &kv : gu_sets)
    WGD_HIP(mv_tune(s, kv.second.data(), (uint32_t)kv.second.size(), 1, qv(m->qx_ffn, H, true, c.epsilon),
                    c.gelu ? MV_GELU : MV_SILU, &to_down));
  for (const auto &kv : dn_sets)
    WGD_HIP(mv_tune(s, kv.second.data(), (uint32_t)kv.second.size(), 1, qv(m->qx_down, F), gemma ? MV_STORE : MV_ADD,
                    gemma ? nullptr : &next));
  return hipSuccess;
}

// Decode step on quantized activations: every matvec reads a QX vector produced by the
// previous kernel; the O and down projections add into the residual stream and re-quantize
// the next RMSNorm's input (x * w; the consumer applies 1/rms from the stored squares).
hipError_t decode_step_q(wgd_model *m, bool advance) {
  const wgd_model_config &c = m->c;
  hipStream_t s = m->ctx->stream;
  const uint32_t H = c.hidden, qd = c.heads * c.head_dim, F = c.intermediate;
  const int32_t *pos = &m->state->pos;
  const bool gemma = is_gemma(m);
  RopeTables rt{};
  if (m->fused_attention) {
    // the model's theta (and scale), and Gemma's local theta (scale 1)
    const uint32_t rot = is_gemma(m) || !c.rotary_dim ? (uint32_t)c.head_dim : (uint32_t)c.rotary_dim;
    rt.half = rot / 2;
    rt.n = is_gemma(m) ? 2 : 1;
    for (uint32_t t = 0; t < rt.n; t++) { rt.freq[t] = m->inv_freq[t]; rt.out[t] = m->rope_cs[t]; }
    rt.scale[0] = c.rope_scale;
    rt.scale[1] = 1.f;
  }
  WGD_HIP(token_start(s, m->embd, &m->state->token, pos, c.embed_scale, m->hidden, m->L[0].attn_norm,
                      qx_view(m->qx_attn, H), rt));
  for (int l = 0; l < c.layers; l++) {
    Layer &L = m->L[l];
    MVTarget qkv[3];
    qkv[0].w = &L.q; qkv[0].y = m->q; qkv[0].bias = L.bq;
    qkv[1].w = &L.k; qkv[1].y = m->k; qkv[1].bias = L.bk;
    qkv[2].w = &L.v; qkv[2].y = m->v; qkv[2].bias = L.bv;
    WGD_HIP(mv_group(s, qkv, 3, qv(m->qx_attn, H, true, c.epsilon)));
    if (m->fused_attention) {
      WGD_HIP(decode_attention_layer(m, l, qx_view(m->qx_o, qd)));
    } else {
      WGD_HIP(attention_block(m, l, 1, 0, pos));
      WGD_HIP(quantize(s, m->att, qd, nullptr, qx_view(m->qx_o, qd)));
    }
    MVOut to_ffn;
    to_ffn.q = qx_view(m->qx_ffn, H); to_ffn.norm_w = L.ffn_norm;
    MVTarget o;
    o.w = &L.o; o.bias = L.bo;
    if (!gemma) {
      o.y = m->hidden;
      WGD_HIP(mv(s, &o, 1, qv(m->qx_o, qd), MV_ADD, &to_ffn));
    } else {
      o.y = m->proj;
      WGD_HIP(mv(s, &o, 1, qv(m->qx_o, qd), MV_STORE));
      WGD_HIP(norm_add_quantize(s, m->proj, L.post_attn, m->hidden, H, c.epsilon, L.ffn_norm, to_ffn.q));
    }
    MVOut to_down;
    to_down.q = qx_view(m->qx_down, F);
    const QXView xf = qv(m->qx_ffn, H, true, c.epsilon);
    if (c.ffn_gate) {
      WGD_HIP(mv(s, L.gate, &L.up, xf, m->prod, c.gelu ? MV_GELU : MV_SILU, &to_down));
    } else {
      WGD_HIP(mv(s, L.up, nullptr, xf, m->up, MV_STORE));
      WGD_HIP(activate(s, m->up, F));
      WGD_HIP(quantize(s, m->up, F, nullptr, to_down.q));
    }
    const bool last = l + 1 == c.layers;
    MVOut next;
    next.q = qx_view(last ? m->qx_head : m->qx_attn, H);
    next.norm_w = last ? m->out_norm : m->L[l + 1].attn_norm;
    if (!gemma) {
      WGD_HIP(mv(s, L.down, nullptr, qv(m->qx_down, F), m->hidden, MV_ADD, &next));
    } else {
      WGD_HIP(mv(s, L.down, nullptr, qv(m->qx_down, F), m->down, MV_STORE));
      WGD_HIP(norm_add_quantize(s, m->down, L.post_ffw, m->hidden, H, c.epsilon, next.norm_w, next.q));
    }
  }
  const Matrix &W = m->have_output && !c.tied_output ? m->output : m->embd;
  MVOut hout;
  hout.arg_part = m->arg_part;
  WGD_HIP(mv(s, W, nullptr, qv(m->qx_head, H, true, c.epsilon), m->logits, MV_STORE, &hout));
  if (m->sampling)
    return sample(s, m->logits, c.vocab, m->sample_params, -1, m->state, m->argmax_buf, m->tokens,
                  (uint32_t)c.context, advance, m->sample_scratch);
  hipLaunchKernelGGL(k_argmax_advance, dim3(1), dim3(256), 0, s, (const uint64_t *)m->arg_part, m->arg_entries,
                     m->argmax_buf, m->state, m->tokens, (uint32_t)m->c.context, advance ? 1 : 0);
  return hipGetLastError();
}

// One decode step with n = 1 for models with a matrix the decode matvec does not read (Q8_0
// or Q4_0 widths off the 64-column planar tile, float rows of a width off 16 elements): the
// batched kernels with the position read from device state.
hipError_t decode_step_generic(wgd_model *m, bool advance) {
  hipStream_t s = m->ctx->stream;
  WGD_HIP(embed_matrix(s, m->embd, &m->state->token, m->hidden, 1, m->c.embed_scale));
  WGD_HIP(layers_batched(m, 1, 0, &m->state->pos));
  WGD_HIP(head(m, 0));
  if (m->sampling)
    return sample(s, m->logits, m->c.vocab, m->sample_params, -1, m->state, m->argmax_buf, m->tokens,
                  (uint32_t)m->c.context, advance, m->sample_scratch);
  if (advance) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, s, m->state, (const int32_t *)m->argmax_buf, m->tokens,
                       (uint32_t)m->c.context);
    WGD_HIP(hipGetLastError());
  }
  return hipSuccess;
}

hipError_t decode_step(wgd_model *m, bool advance) {
  return m->qpath ? decode_step_q(m, advance) : decode_step_generic(m, advance);
}

int validate_ids(wgd_model *m, const int32_t *ids, int32_t n) {
  for (int i = 0; i < n; i++)
    if (ids[i] < 0 || ids[i] >= m->c.vocab)
      return fail(m->ctx, WGD_E_INVALID, "token id %d outside the %d-entry vocabulary", ids[i], m->c.vocab);
  return WGD_OK;
}

int need_tensor(wgd_model *m, bool have, const char *name) {
  return have ? WGD_OK : fail(m->ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name);
}

}  // namespace

void wgd::model_destroy(wgd_model *m) {
  if (!m) return;
  wgd_context *ctx = m->ctx;
  hipStreamSynchronize(ctx->stream);
  if (m->exec) hipGraphExecDestroy(m->exec);
  if (m->graph) hipGraphDestroy(m->graph);
  if (m->exec_s) hipGraphExecDestroy(m->exec_s);
  if (m->graph_s) hipGraphDestroy(m->graph_s);
  for (void *p : m->owned) ctx_free(ctx, p);
  ctx->models.erase(m);
  delete m;
}

extern "C" {

int wgd_model_create(wgd_context *ctx, const wgd_model_config *cfg, const int32_t *capacities, wgd_model **out) {
  if (!ctx || !cfg || !capacities || !out) return fail(ctx, WGD_E_INVALID, "wgd_model_create: NULL argument");
  hipSetDevice(ctx->device);
  *out = nullptr;
  const wgd_model_config &c = *cfg;
  if (c.layers < 1 || c.layers > 128 || c.hidden < 1 || c.hidden > 16384 || c.heads < 1 || c.heads > 256 ||
      c.kv_heads < 1 || c.heads % c.kv_heads || c.head_dim < 2 || c.head_dim > 512 || c.head_dim % 2 ||
      c.intermediate < 1 || c.intermediate > 131072 || c.vocab < 1 || c.vocab > 1000000 || c.rotary_dim % 2 ||
      c.rotary_dim > c.head_dim || c.context < 1 || c.batch < 1 || c.batch > 128 || c.heads / c.kv_heads > 16 ||
      (c.family != 0 && c.family != 1) || c.window < 0 || c.period < 0 || (c.kv_f16 != 0 && c.kv_f16 != 1))
    return fail(ctx, WGD_E_INVALID, "Unsupported model dimensions.");
  wgd_model *m = new wgd_model();
  m->ctx = ctx;
  m->c = c;
  m->L.resize(c.layers);
  m->seen.assign(c.layers, 0);
  ctx->models.insert(m);
  const uint64_t B = c.batch, H = c.hidden, qd = (uint64_t)c.heads * c.head_dim, kd = (uint64_t)c.kv_heads * c.head_dim,
                 F = c.intermediate;
  int rc = WGD_OK;
  rc = rc ? rc : alloc_t(m, B * H, "hidden", &m->hidden);
  rc = rc ? rc : alloc_t(m, B * H, "normed", &m->normed);
  rc = rc ? rc : alloc_t(m, B * qd, "q", &m->q);
  rc = rc ? rc : alloc_t(m, B * kd, "k", &m->k);
  rc = rc ? rc : alloc_t(m, B * kd, "v", &m->v);
  rc = rc ? rc : alloc_t(m, B * qd, "attention", &m->att);
  rc = rc ? rc : alloc_t(m, B * H, "projection", &m->proj);
  rc = rc ? rc : alloc_t(m, B * F, "gate", &m->gate);
  rc = rc ? rc : alloc_t(m, B * F, "up", &m->up);
  rc = rc ? rc : alloc_t(m, B * F, "product", &m->prod);
  rc = rc ? rc : alloc_t(m, B * H, "down", &m->down);
  rc = rc ? rc : alloc_t(m, B * residual_split_segs((uint32_t)H), "deferred norm sums", &m->res_sq);
  rc = rc ? rc : alloc_t(m, (uint64_t)c.vocab, "logits", &m->logits);
  rc = rc ? rc : alloc_t(m, B, "ids", &m->ids);
  rc = rc ? rc : alloc_t(m, 1, "step state", &m->state);
  rc = rc ? rc : alloc_t(m, (uint64_t)c.context + 1, "decode tokens", &m->tokens);
  rc = rc ? rc : alloc_t(m, 2 + 2 * 256, "argmax", &m->argmax_buf);
  rc = rc ? rc : alloc_t(m, 1, "sampling settings", &m->sample_params);
  rc = rc ? rc : alloc(m, sample_scratch_bytes((uint32_t)c.vocab), "sampling candidates", &m->sample_scratch);
  m->att_part_floats = attention_scratch_floats(c.heads, c.head_dim, 1, (uint32_t)device_cu_count() * 4);
  if (decode_attention_supported(c.heads, c.kv_heads, c.head_dim))
    for (int l = 0; l < c.layers; l++)
      if (capacities[l] > 0)
        m->att_part_floats = std::max(m->att_part_floats, decode_attention_scratch_floats(c.heads, c.kv_heads, c.head_dim,
                                                                                          (uint32_t)capacities[l]));
  rc = rc ? rc : alloc_t(m, m->att_part_floats, "attention split scratch", &m->att_part);
  for (int l = 0; !rc && l < c.layers; l++) {
    if (capacities[l] < 1) { rc = fail(ctx, WGD_E_INVALID, "layer %d: KV capacity %d", l, capacities[l]); break; }
    m->L[l].cap = (uint32_t)capacities[l];
    char label[64];
    snprintf(label, sizeof label, "K %d", l);
    const uint64_t ring = (uint64_t)capacities[l] * kd * (c.kv_f16 ? 2 : 4);
    rc = alloc(m, ring, label, &m->L[l].kc);
    snprintf(label, sizeof label, "V %d", l);
    rc = rc ? rc : alloc(m, ring, label, &m->L[l].vc);
  }
  if (rc) { std::string e = ctx->error; model_destroy(m); ctx->error = e; return rc; }
  *out = m;
  return WGD_OK;
}

int wgd_model_tensor(wgd_model *m, const char *name, int32_t type, int32_t n_dims, const uint64_t *dims,
                     const void *data, uint64_t bytes) {
  if (!m || !name || !dims || !data) return fail(m ? m->ctx : nullptr, WGD_E_INVALID, "wgd_model_tensor: NULL argument");
  wgd_context *ctx = m->ctx;
  hipSetDevice(ctx->device);
  if (m->ready) return fail(ctx, WGD_E_STATE, "wgd_model_tensor: model is already sealed");
  if (block_size(type) == 0) return fail(ctx, WGD_E_INVALID, "Unsupported tensor quantization %d in %s.", type, name);
  if (n_dims < 1 || n_dims > 2) return fail(ctx, WGD_E_INVALID, "%s: %d dimensions", name, n_dims);
  const uint64_t ne0 = dims[0], ne1 = n_dims == 2 ? dims[1] : 1;
  if (!ne0 || !ne1 || ne0 % block_size(type)) return fail(ctx, WGD_E_INVALID, "Invalid shape for %s.", name);
  const uint64_t need = ne1 * row_bytes(type, ne0);
  if (bytes != need) return fail(ctx, WGD_E_INVALID, "%s: %llu bytes given, shape needs %llu", name, (unsigned long long)bytes, (unsigned long long)need);

  // Route the name to its slot.
  int layer = -1, slot = -1;
  bool embd = false, outw = false, onorm = false;
  if (!strcmp(name, "token_embd.weight")) embd = true;
  else if (!strcmp(name, "output.weight")) outw = true;
  else if (!strcmp(name, "output_norm.weight")) onorm = true;
  else {
    int l = -1, used = 0;
    if (sscanf(name, "blk.%d.%n", &l, &used) == 1 && used > 0 && l >= 0 && l < m->c.layers) {
      for (int k = 0; k < S_COUNT; k++) if (!strcmp(name + used, kSlotNames[k])) { layer = l; slot = k; break; }
    }
    if (slot < 0) return WGD_OK;  // tensors outside the dense path are ignored (engine.ts reads by name)
  }
  const bool vec = n_dims == 1;
  char label[160];
  snprintf(label, sizeof label, "%s", name);
  hipStream_t s = ctx->stream;
  if (vec) {
    if (embd || outw) return fail(ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name);
    void *raw = nullptr; float *f = nullptr;
    int rc = ctx_alloc(ctx, need, "upload staging", &raw);
    if (rc) return rc;
    rc = alloc_t(m, ne0, label, &f);
    if (!rc) rc = ctx_check(ctx, hipMemcpyAsync(raw, data, need, hipMemcpyHostToDevice, s), name);
    if (!rc) rc = ctx_check(ctx, dequant(s, type, (const uint8_t *)raw, f, ne0), name);
    if (!rc) rc = ctx_sync(ctx, name);
    ctx_free(ctx, raw);
    if (rc) return rc;
    if (onorm) { if (ne0 != (uint64_t)m->c.hidden) return fail(ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name); m->out_norm = f; return WGD_OK; }
    Layer &L = m->L[layer];
    float **dst = nullptr;
    uint64_t want = 0;
    const uint64_t H = m->c.hidden, qd = (uint64_t)m->c.heads * m->c.head_dim, kd = (uint64_t)m->c.kv_heads * m->c.head_dim;
    switch (slot) {
      case S_ATTN_NORM: dst = &L.attn_norm; want = H; break;
      case S_FFN_NORM: dst = &L.ffn_norm; want = H; break;
      case S_POST_ATTN: dst = &L.post_attn; want = H; break;
      case S_POST_FFW: dst = &L.post_ffw; want = H; break;
      case S_QN: dst = &L.q_norm; want = m->c.head_dim; break;
      case S_KN: dst = &L.k_norm; want = m->c.head_dim; break;
      case S_QB: dst = &L.bq; want = qd; break;
      case S_KB: dst = &L.bk; want = kd; break;
      case S_VB: dst = &L.bv; want = kd; break;
      case S_OB: dst = &L.bo; want = H; break;
      default: return fail(ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name);
    }
    if (ne0 != want) return fail(ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name);
    *dst = f;
    m->seen[layer] |= 1u << slot;
    return WGD_OK;
  }
  // Matrices: GGUF bytes kept as-is, or rewritten to the planar layout.
  if (ne0 > 0xFFFFFFFFull || ne1 > 0xFFFFFFFFull) return fail(ctx, WGD_E_INVALID, "%s: too large", name);
  Matrix mat; mat.type = type; mat.cols = (uint32_t)ne0; mat.rows = (uint32_t)ne1;
  void *dev = nullptr;
  int rc = alloc(m, has_planar(type, mat.cols) ? planar_bytes(type, mat.cols, mat.rows) : need, label, &dev);
  if (rc) return rc;
  if (has_planar(type, mat.cols)) {
    void *raw = nullptr;
    rc = ctx_alloc(ctx, need, "upload staging", &raw);
    if (rc) return rc;
    rc = ctx_check(ctx, hipMemcpyAsync(raw, data, need, hipMemcpyHostToDevice, s), name);
    if (!rc) rc = ctx_check(ctx, repack_planar(s, type, (const uint8_t *)raw, (uint8_t *)dev, mat.cols, mat.rows), name);
    if (!rc) rc = ctx_sync(ctx, name);
    ctx_free(ctx, raw);
    if (rc) return rc;
    mat.layout = LAYOUT_PLANAR;
  } else {
    rc = ctx_check(ctx, hipMemcpyAsync(dev, data, need, hipMemcpyHostToDevice, s), name);
    if (!rc) rc = ctx_sync(ctx, name);
    if (rc) return rc;
    mat.layout = LAYOUT_GGUF;
  }
  mat.data = (const uint8_t *)dev;
  const wgd_model_config &c = m->c;
  const uint32_t H = c.hidden, qd = c.heads * c.head_dim, kd = c.kv_heads * c.head_dim, F = c.intermediate;
  auto shape_ok = [&](uint32_t cols, uint32_t rows) { return mat.cols == cols && mat.rows == rows; };
  if (embd) { if (!shape_ok(H, c.vocab)) return fail(ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name); m->embd = mat; m->have_embd = true; return WGD_OK; }
  if (outw) { if (!shape_ok(H, c.vocab)) return fail(ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name); m->output = mat; m->have_output = true; return WGD_OK; }
  Layer &L = m->L[layer];
  bool ok = false;
  switch (slot) {
    case S_Q: ok = shape_ok(H, qd); L.q = mat; break;
    case S_K: ok = shape_ok(H, kd); L.k = mat; break;
    case S_V: ok = shape_ok(H, kd); L.v = mat; break;
    case S_O: ok = shape_ok(qd, H); L.o = mat; break;
    case S_GATE: ok = shape_ok(H, F); L.gate = mat; break;
    case S_UP: ok = shape_ok(H, F); L.up = mat; break;
    case S_DOWN: ok = shape_ok(F, H); L.down = mat; break;
    default: ok = false;
  }
  if (!ok) return fail(ctx, WGD_E_INVALID, "Missing or invalid tensor %s.", name);
  m->seen[layer] |= 1u << slot;
  return WGD_OK;
}

int wgd_model_ready(wgd_model *m) {
  if (!m) return fail(nullptr, WGD_E_INVALID, "wgd_model_ready: NULL model");
  wgd_context *ctx = m->ctx;
  const wgd_model_config &c = m->c;
  int rc = need_tensor(m, m->have_embd, "token_embd.weight");
  rc = rc ? rc : need_tensor(m, m->out_norm != nullptr, "output_norm.weight");
  if (!rc && !c.tied_output) rc = need_tensor(m, m->have_output, "output.weight");
  for (int l = 0; !rc && l < c.layers; l++) {
    std::vector<int> req = {S_ATTN_NORM, S_Q, S_K, S_V, S_O, S_FFN_NORM, S_UP, S_DOWN};
    if (c.ffn_gate) req.push_back(S_GATE);
    if (c.qk_norm || c.family == 1) { req.push_back(S_QN); req.push_back(S_KN); }
    if (c.family == 1) { req.push_back(S_POST_ATTN); req.push_back(S_POST_FFW); }
    if (c.bias_q) req.push_back(S_QB);
    if (c.bias_k) req.push_back(S_KB);
    if (c.bias_v) req.push_back(S_VB);
    if (c.bias_output) req.push_back(S_OB);
    for (int sl : req)
      if (!(m->seen[l] & (1u << sl))) {
        char name[96];
        snprintf(name, sizeof name, "blk.%d.%s", l, kSlotNames[sl]);
        rc = need_tensor(m, false, name);
        break;
      }
  }
  if (rc) return rc;
  // prompt GEMM scratch: split-K sums and the bf16 split input, the most any layer matrix
  // uses at the batch size
  uint64_t gp = 0, gx = 0;
  for (const Layer &L : m->L) {
    for (const Matrix *w : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down})
      if (w->data) {
        gp = std::max(gp, gemm_split_floats(*w, (uint32_t)c.batch));
        gx = std::max(gx, gemm_input_elems(w->cols, (uint32_t)c.batch));
      }
    gp = std::max(gp, gemm_group_split_floats(qkv_group(m, L), (uint32_t)c.batch));
    if (L.o.data) gp = std::max(gp, gemm_group_split_floats(res_group(m, L.o), (uint32_t)c.batch));
    if (L.down.data) gp = std::max(gp, gemm_group_split_floats(res_group(m, L.down), (uint32_t)c.batch));
    if (c.ffn_gate) gp = std::max(gp, gemm_group_split_floats(glu_group(m, L), (uint32_t)c.batch));
  }
  if (gp && !m->gemm_part.p) {
    rc = alloc_t(m, gp, "prompt GEMM split sums", &m->gemm_part.p);
    if (rc) return rc;
    m->gemm_part.floats = gp;
  }
  if (gx && !m->gemm_part.xs) {
    rc = alloc_t(m, gx, "prompt GEMM split input", &m->gemm_part.xs);
    if (rc) return rc;
    m->gemm_part.xs_elems = gx;
  }
  // a prompt batch's RoPE rotations (the model's theta; Gemma's local theta too)
  if (!m->rope_batch[0]) {
    const uint32_t rot = is_gemma(m) || !c.rotary_dim ? (uint32_t)c.head_dim : (uint32_t)c.rotary_dim;
    const uint64_t entries = (uint64_t)c.batch * (rot / 2);
    rc = alloc_t(m, entries, "rope batch table", &m->rope_batch[0]);
    if (!rc && is_gemma(m)) rc = alloc_t(m, entries, "rope batch table (local)", &m->rope_batch[1]);
    if (rc) return rc;
  }
  // The quantized decode path needs every matrix in a type the integer matvec reads.
  const Matrix &head_w = m->have_output && !c.tied_output ? m->output : m->embd;
  bool q = mv_supported(head_w);
  for (int l = 0; q && l < c.layers; l++) {
    const Layer &L = m->L[l];
    q = mv_supported(L.q) && mv_supported(L.k) && mv_supported(L.v) && mv_supported(L.o) &&
        mv_supported(L.up) && mv_supported(L.down) &&
        (!c.ffn_gate || (mv_supported(L.gate) && L.gate.type == L.up.type && L.gate.layout == L.up.layout));
  }
  if (q) {
    const uint32_t H = c.hidden, qd = c.heads * c.head_dim, F = c.intermediate;
    rc = alloc(m, qx_bytes(H), "qx attn", &m->qx_attn);
    rc = rc ? rc : alloc(m, qx_bytes(H), "qx ffn", &m->qx_ffn);
    rc = rc ? rc : alloc(m, qx_bytes(qd), "qx o", &m->qx_o);
    rc = rc ? rc : alloc(m, qx_bytes(F), "qx down", &m->qx_down);
    rc = rc ? rc : alloc(m, qx_bytes(H), "qx head", &m->qx_head);
    m->arg_entries = mv_arg_entries(head_w);
    rc = rc ? rc : alloc_t(m, m->arg_entries, "head argmax keys", &m->arg_part);
    if (rc) return rc;
    m->qpath = true;
    const bool norms = !(is_gemma(m) || c.qk_norm) || [&] {
      for (const Layer &L : m->L) if (!L.q_norm || !L.k_norm) return false;
      return true;
    }();
    m->fused_attention = decode_attention_supported(c.heads, c.kv_heads, c.head_dim) && norms;
    if (m->fused_attention) {
      // one table per distinct theta: the model's, and Gemma's local layers'
      const uint32_t rot = is_gemma(m) || !c.rotary_dim ? (uint32_t)c.head_dim : (uint32_t)c.rotary_dim;
      rc = alloc_t(m, rot / 2, "rope frequencies", &m->inv_freq[0]);
      if (!rc) rc = ctx_check(ctx, rope_inv_freq(ctx->stream, m->inv_freq[0], rot, c.theta), "rope frequencies");
      if (!rc) rc = alloc_t(m, rot, "rope table", &m->rope_cs[0]);
      if (!rc && is_gemma(m)) {
        rc = alloc_t(m, rot / 2, "rope frequencies (local)", &m->inv_freq[1]);
        if (!rc) rc = ctx_check(ctx, rope_inv_freq(ctx->stream, m->inv_freq[1], rot, c.local_theta), "rope frequencies");
        if (!rc) rc = alloc_t(m, rot, "rope table (local)", &m->rope_cs[1]);
      }
      if (rc) return rc;
    }
    rc = ctx_check(ctx, tune_decode(m), "decode launch shapes");
    if (rc) return rc;
  }
  m->ready = true;
  return ctx_sync(ctx, "model upload");
}

int wgd_model_forward(wgd_model *m, const int32_t *ids, int32_t n, int32_t start, float *logits, int32_t *argmax_out) {
  if (!m) return fail(nullptr, WGD_E_INVALID, "wgd_model_forward: NULL model");
  wgd_context *ctx = m->ctx;
  hipSetDevice(ctx->device);
  if (!m->ready) return fail(ctx, WGD_E_STATE, "Load a model first.");
  if (!ids || n < 1 || n > m->c.batch || start < 0) return fail(ctx, WGD_E_INVALID, "forward: %d tokens at %d (batch %d)", n, start, m->c.batch);
  // positions past the context would wrap the full-context rings onto live keys
  if ((int64_t)start + n > m->c.context)
    return fail(ctx, WGD_E_INVALID, "forward: positions %d..%d outside the context of %d", start, start + n - 1, m->c.context);
  int rc = validate_ids(m, ids, n);
  if (rc) return rc;
  hipStream_t s = ctx->stream;
  const bool want = logits || argmax_out;
  if (n == 1) {
    StepState st = {start, ids[0], 0, 0};
    rc = ctx_check(ctx, hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s), "forward");
    if (!rc) rc = ctx_check(ctx, decode_step(m, false), "forward");
  } else {
    rc = ctx_check(ctx, hipMemcpyAsync(m->ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, s), "forward");
    if (!rc) rc = ctx_check(ctx, embed_matrix(s, m->embd, m->ids, m->hidden, n, m->c.embed_scale), "embed");
    if (!rc) rc = ctx_check(ctx, layers_batched(m, (uint32_t)n, (uint32_t)start), "forward");
    if (!rc && want) rc = ctx_check(ctx, head(m, (uint32_t)n - 1), "head");
    // the next token takes position start + n
    if (!rc && want && m->sampling)
      rc = ctx_check(ctx, sample(s, m->logits, m->c.vocab, m->sample_params, start + n, nullptr, m->argmax_buf, nullptr, 0,
                                 false, m->sample_scratch), "sample");
  }
  if (!rc) rc = ctx_sync(ctx, "GPU fault during forward");
  if (rc) return rc;
  if (logits) {
    hipError_t e = hipMemcpy(logits, m->logits, sizeof(float) * m->c.vocab, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(ctx, e, "logits read-back");
  }
  if (argmax_out) {
    int32_t id = -1;
    hipError_t e = hipMemcpy(&id, m->argmax_buf, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(ctx, e, "argmax read-back");
    *argmax_out = id;
    if (id < 0) return fail(ctx, WGD_E_NONFINITE, "Inference produced non-finite logits. Stop and report this model/runtime combination.");
  }
  return WGD_OK;
}

int wgd_model_decode(wgd_model *m, int32_t token, int32_t start, int32_t count, int32_t *out_tokens) {
  if (!m) return fail(nullptr, WGD_E_INVALID, "wgd_model_decode: NULL model");
  wgd_context *ctx = m->ctx;
  hipSetDevice(ctx->device);
  if (!m->ready) return fail(ctx, WGD_E_STATE, "Load a model first.");
  if (count < 0 || start < 0 || !out_tokens) return fail(ctx, WGD_E_INVALID, "decode: bad arguments");
  if (count == 0) return WGD_OK;
  if ((int64_t)start + count > m->c.context) return fail(ctx, WGD_E_INVALID, "decode: %d tokens from position %d exceed the %d-token context", count, start, m->c.context);
  int rc = validate_ids(m, &token, 1);
  if (rc) return rc;
  hipStream_t s = ctx->stream;
  StepState st = {start, token, 0, 0};
  rc = ctx_check(ctx, hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s), "decode");
  if (rc) return rc;
  hipGraph_t &graph = m->sampling ? m->graph_s : m->graph;
  hipGraphExec_t &exec = m->sampling ? m->exec_s : m->exec;
  if (!exec) {
    // Run one step eagerly first: it validates every launch outside capture.
    rc = ctx_check(ctx, decode_step(m, true), "decode");
    if (!rc) rc = ctx_sync(ctx, "GPU fault during decode");
    if (rc) return rc;
    rc = ctx_check(ctx, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "graph capture");
    if (rc) return rc;
    hipError_t e = decode_step(m, true);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(s, &g);
    if (e != hipSuccess || e2 != hipSuccess) { if (g) hipGraphDestroy(g); return hip_fail(ctx, e != hipSuccess ? e : e2, "graph capture"); }
    graph = g;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) { exec = nullptr; return hip_fail(ctx, e, "graph instantiate"); }
    for (int32_t i = 1; i < count; i++) {
      e = hipGraphLaunch(exec, s);
      if (e != hipSuccess) return hip_fail(ctx, e, "graph launch");
    }
  } else {
    for (int32_t i = 0; i < count; i++) {
      hipError_t e = hipGraphLaunch(exec, s);
      if (e != hipSuccess) return hip_fail(ctx, e, "graph launch");
    }
  }
  rc = ctx_sync(ctx, "GPU fault during decode");
  if (rc) return rc;
  StepState fin;
  hipError_t e = hipMemcpy(&fin, m->state, sizeof fin, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(ctx, e, "decode state");
  e = hipMemcpy(out_tokens, m->tokens, sizeof(int32_t) * count, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(ctx, e, "decode tokens");
  if (fin.error) return fail(ctx, WGD_E_NONFINITE, "Inference produced non-finite logits. Stop and report this model/runtime combination.");
  return WGD_OK;
}

int wgd_model_attention_timing(wgd_model *m, int32_t layer, int32_t pos, int32_t reps, double *us) {
  if (!m || !us) return fail(m ? m->ctx : nullptr, WGD_E_INVALID, "wgd_model_attention_timing: NULL argument");
  wgd_context *ctx = m->ctx;
  hipSetDevice(ctx->device);
  if (!m->ready) return fail(ctx, WGD_E_STATE, "Load a model first.");
  if (!m->qpath || !m->fused_attention)
    return fail(ctx, WGD_E_INVALID, "attention_timing: this model's decode step has no fused attention launch");
  if (layer < 0 || layer >= m->c.layers || pos < 0 || pos >= m->c.context || reps < 1 || reps > 100000)
    return fail(ctx, WGD_E_INVALID, "attention_timing: layer %d, position %d, %d repetitions", layer, pos, reps);
  hipStream_t s = ctx->stream;
  StepState st = {pos, 0, 0, 0};
  int rc = ctx_check(ctx, hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s), "attention_timing");
  const QXOut qx = qx_view(m->qx_o, (uint32_t)(m->c.heads * m->c.head_dim));
  if (!rc) rc = ctx_check(ctx, decode_attention_layer(m, layer, qx), "attention_timing");  // warm
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (!rc) rc = ctx_check(ctx, hipEventCreate(&e0), "attention_timing");
  if (!rc) rc = ctx_check(ctx, hipEventCreate(&e1), "attention_timing");
  if (!rc) rc = ctx_check(ctx, hipEventRecord(e0, s), "attention_timing");
  for (int32_t i = 0; !rc && i < reps; i++) rc = ctx_check(ctx, decode_attention_layer(m, layer, qx), "attention_timing");
  if (!rc) rc = ctx_check(ctx, hipEventRecord(e1, s), "attention_timing");
  if (!rc) rc = ctx_sync(ctx, "GPU fault during attention timing");
  float ms = 0.f;
  if (!rc) rc = ctx_check(ctx, hipEventElapsedTime(&ms, e0, e1), "attention_timing");
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  if (!rc) *us = (double)ms * 1e3 / reps;
  return rc;
}

int wgd_model_sampling(wgd_model *m, double temperature, uint32_t top_k, double top_p, uint64_t seed) {
  if (!m) return fail(nullptr, WGD_E_INVALID, "wgd_model_sampling: NULL model");
  wgd_context *ctx = m->ctx;
  hipSetDevice(ctx->device);
  // engine.ts:262-264
  if (!(temperature >= 0.0 && temperature <= 2.0) || top_k < 1 || top_k > 200 || !(top_p > 0.0 && top_p <= 1.0))
    return fail(ctx, WGD_E_INVALID, "Invalid sampling settings.");
  const SampleParams p = {temperature, top_p, top_k, 0, seed};
  hipError_t e = hipMemcpyAsync(m->sample_params, &p, sizeof p, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "sampling settings");
  int rc = ctx_sync(ctx, "sampling settings");
  if (rc) return rc;
  m->sampling = temperature != 0.0;
  return WGD_OK;
}

void wgd_model_destroy(wgd_model *m) {
  if (!m) return;
  hipSetDevice(m->ctx->device);
  model_destroy(m);
}

}  // extern "C"
