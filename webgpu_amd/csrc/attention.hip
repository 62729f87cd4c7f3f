// attention.hip — causal GQA attention over the f32 KV ring, split-K (gfx950).
//
// Semantics of attentionShader (src/core/shaders.ts:88-122): for query token b and head h,
// keys t in [end - min(end, window), end) with end = start + b + 1, read from ring slot
// t % capacity of a [capacity][kvHeads][hd] cache, kv head h / (heads / kvHeads), scores
// scale * q.k, softmax-weighted sum of V.
//
// The reference runs one 64-lane workgroup per (head, query) serially over every key. Here a
// workgroup owns one kv head, a block of queries and a contiguous chunk of the key range:
// every (query, head) row that shares the kv head reuses the same K/V tile staged in LDS,
// and the key range is split across workgroups (flash-decoding) so decode at long context
// spreads over the whole chip. Each split keeps an online-softmax state (m, l, O) and a
// second kernel merges the splits. Tile size T keeps T*hd = 4096 floats per operand.
#include "internal.h"
#include "decode.h"
#include "attention.h"
#include "split.h"

namespace wgd {

struct AttnK {
  const float *q; const void *k, *v; float *y, *part;  // k, v: ring of E elements
  uint32_t heads, kvh, hd, start; const int32_t *start_dev;
  float scale; uint32_t window, capacity, batch;
  uint32_t qb, nsplit, T, R, group;
};

constexpr int ATT_MAX_PER_THREAD = 32;  // R*hd/256 with R <= 16, hd <= 512

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

template <class E>
__global__ __launch_bounds__(256) void k_attention(AttnK a) {
  extern __shared__ float lds[];
  const uint32_t hd = a.hd, T = a.T, R = a.R, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float *Ks = lds;                         // [T][hd+1]
  float *Vs = Ks + T * (hd + 1);           // [T][hd]
  float *Qs = Vs + T * hd;                 // [R][hd]
  float *S = Qs + R * hd;                  // [R][T]
  float *mrow = S + R * T, *lrow = mrow + R, *corr = lrow + R;

  const uint32_t kv = blockIdx.x, b0 = blockIdx.y * a.qb, z = blockIdx.z;
  const uint32_t nq = a.batch - b0 < a.qb ? a.batch - b0 : a.qb;
  const uint32_t s0 = a.start_dev ? (uint32_t)*a.start_dev : a.start;
  const uint32_t first_end = s0 + b0 + 1, last_end = s0 + b0 + nq;
  const uint32_t begin0 = first_end - (first_end < a.window ? first_end : a.window);
  const uint32_t range = last_end - begin0;
  uint32_t chunk = (range + a.nsplit - 1) / a.nsplit;
  chunk = (chunk + T - 1) / T * T;
  const uint32_t lo = begin0 + z * chunk;
  const uint32_t hi = lo + chunk < last_end ? lo + chunk : last_end;

  for (uint32_t i = tid; i < R * hd; i += 256) {
    uint32_t r = i / hd, d = i % hd, qi = r / a.group, h = kv * a.group + r % a.group;
    Qs[i] = qi < nq ? a.q[((uint64_t)(b0 + qi) * a.heads + h) * hd + d] : 0.f;
  }
  if (tid < R) { mrow[tid] = -INFINITY; lrow[tid] = 0.f; }
  const uint32_t per = (R * hd + 255) / 256;
  float o[ATT_MAX_PER_THREAD];
#pragma unroll
  for (int i = 0; i < ATT_MAX_PER_THREAD; i++) o[i] = 0.f;

  for (uint32_t t0 = lo; t0 < hi; t0 += T) {
    __syncthreads();
    for (uint32_t i = tid; i < T * hd; i += 256) {
      uint32_t j = i / hd, d = i % hd, t = t0 + j;
      float kvk = 0.f, kvv = 0.f;
      if (t < hi) {
        uint64_t src = ((uint64_t)(t % a.capacity) * a.kvh + kv) * hd + d;
        kvk = kv_get<E>(a.k, src); kvv = kv_get<E>(a.v, src);
      }
      Ks[j * (hd + 1) + d] = kvk;
      Vs[j * hd + d] = kvv;
    }
    __syncthreads();
    for (uint32_t p = tid; p < R * T; p += 256) {
      uint32_t r = p / T, j = p % T, t = t0 + j, qi = r / a.group;
      float sc = -INFINITY;
      if (qi < nq && t < hi) {
        uint32_t end = s0 + b0 + qi + 1, begin = end - (end < a.window ? end : a.window);
        if (t >= begin && t < end) {
          const float *qr = Qs + r * hd, *kr = Ks + j * (hd + 1);
          float dot = 0.f;
          for (uint32_t d = 0; d < hd; d++) dot += qr[d] * kr[d];
          sc = dot * a.scale;
        }
      }
      S[p] = sc;
    }
    __syncthreads();
    for (uint32_t r = wv; r < R; r += 4) {
      float mx = -INFINITY;
      for (uint32_t j = lane; j < T; j += 64) mx = fmaxf(mx, S[r * T + j]);
      mx = wave_max(mx);
      float m_old = mrow[r], m_new = fmaxf(m_old, mx);
      float sum = 0.f;
      for (uint32_t j = lane; j < T; j += 64) {
        float sv = S[r * T + j];
        float pv = (m_new == -INFINITY || sv == -INFINITY) ? 0.f : expf(sv - m_new);
        S[r * T + j] = pv;
        sum += pv;
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        float c = (m_old == -INFINITY) ? 0.f : expf(m_old - m_new);
        if (m_new == -INFINITY) c = 1.f;
        corr[r] = c;
        lrow[r] = lrow[r] * c + sum;
        mrow[r] = m_new;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ATT_MAX_PER_THREAD; i++) {
      if ((uint32_t)i >= per) break;
      uint32_t e = tid + 256 * i;
      if (e >= R * hd) break;
      uint32_t r = e / hd, d = e % hd;
      float acc = o[i] * corr[r];
      const float *pr = S + r * T;
      for (uint32_t j = 0; j < T; j++) acc += pr[j] * Vs[j * hd + d];
      o[i] = acc;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ATT_MAX_PER_THREAD; i++) {
    if ((uint32_t)i >= per) break;
    uint32_t e = tid + 256 * i;
    if (e >= R * hd) break;
    uint32_t r = e / hd, d = e % hd, qi = r / a.group, h = kv * a.group + r % a.group;
    if (qi >= nq) continue;
    uint64_t row = (uint64_t)(b0 + qi) * a.heads + h;
    if (a.nsplit == 1) {
      a.y[row * hd + d] = o[i] / lrow[r];
    } else {
      float *pp = a.part + ((uint64_t)z * a.batch * a.heads + row) * (hd + 2);
      if (d == 0) { pp[0] = mrow[r]; pp[1] = lrow[r]; }
      pp[2 + d] = o[i];
    }
  }
}

// With xs set (hd % 8 == 0, heads * hd % 64 == 0), the output row is also written in the
// prompt GEMM's split form for the O projection (row = token * heads + head).
__global__ __launch_bounds__(128) void k_attention_combine(const float *part, float *y, uint32_t rows,
                                                           uint32_t hd, uint32_t nsplit, uint16_t *xs, uint32_t heads) {
  __shared__ float out[512];
  const uint64_t row = blockIdx.x;
  const uint64_t stride = (uint64_t)rows * (hd + 2);
  float M = -INFINITY;
  for (uint32_t z = 0; z < nsplit; z++) M = fmaxf(M, part[z * stride + row * (hd + 2)]);
  float L = 0.f;
  for (uint32_t z = 0; z < nsplit; z++) {
    const float *pp = part + z * stride + row * (hd + 2);
    if (pp[0] != -INFINITY) L += pp[1] * expf(pp[0] - M);
  }
  for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    for (uint32_t z = 0; z < nsplit; z++) {
      const float *pp = part + z * stride + row * (hd + 2);
      if (pp[0] != -INFINITY) acc += pp[2 + d] * expf(pp[0] - M);
    }
    const float o = L > 0.f ? acc / L : 0.f;
    y[row * hd + d] = o;
    out[d] = o;
  }
  if (!xs) return;
  __syncthreads();
  const uint32_t tok = (uint32_t)(row / heads), h = (uint32_t)(row % heads);
  for (uint32_t g = threadIdx.x; g < hd / 8; g += blockDim.x)
    split_store8(xs, heads * hd, tok, h * hd + 8 * g, make_float4(out[8 * g], out[8 * g + 1], out[8 * g + 2], out[8 * g + 3]),
                 make_float4(out[8 * g + 4], out[8 * g + 5], out[8 * g + 6], out[8 * g + 7]));
}

// k_attention_combine for at most S splits, the same arithmetic in the same order, with each
// pass's loads over the splits issued together (raw buffer loads over the partials, zero
// past the last split, which selects leave out).
template <uint32_t S>
__global__ __launch_bounds__(128) void k_attention_combine_s(const float *part, float *y, uint32_t rows, uint32_t hd,
                                                             uint32_t nsplit, uint16_t *xs, uint32_t heads) {
  __shared__ float out[512];
  const uint64_t row = blockIdx.x;
  const uint64_t stride = (uint64_t)rows * (hd + 2);
  const __amdgpu_buffer_rsrc_t rp = split_rsrc(part, nsplit, stride);
  const uint32_t sb = (uint32_t)(4 * stride), rb = (uint32_t)(4 * row * (hd + 2));
  float mz[S], lz[S];
#pragma unroll
  for (uint32_t z = 0; z < S; z++) {
    mz[z] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, rb + z * sb, 0, 0));
    lz[z] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, rb + z * sb + 4, 0, 0));
  }
  float M = -INFINITY;
#pragma unroll
  for (uint32_t z = 0; z < S; z++) M = z < nsplit ? fmaxf(M, mz[z]) : M;
  bool use[S];
  float wz[S];
  float L = 0.f;
#pragma unroll
  for (uint32_t z = 0; z < S; z++) {
    use[z] = z < nsplit && mz[z] != -INFINITY;
    wz[z] = use[z] ? expf(mz[z] - M) : 0.f;
    L = use[z] ? L + lz[z] * wz[z] : L;
  }
  for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
    float pz[S];
#pragma unroll
    for (uint32_t z = 0; z < S; z++)
      pz[z] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, rb + z * sb + 4 * (2 + d), 0, 0));
    float acc = 0.f;
#pragma unroll
    for (uint32_t z = 0; z < S; z++) acc = use[z] ? acc + pz[z] * wz[z] : acc;
    const float o = L > 0.f ? acc / L : 0.f;
    y[row * hd + d] = o;
    out[d] = o;
  }
  if (!xs) return;
  __syncthreads();
  const uint32_t tok = (uint32_t)(row / heads), h = (uint32_t)(row % heads);
  for (uint32_t g = threadIdx.x; g < hd / 8; g += blockDim.x)
    split_store8(xs, heads * hd, tok, h * hd + 8 * g, make_float4(out[8 * g], out[8 * g + 1], out[8 * g + 2], out[8 * g + 3]),
                 make_float4(out[8 * g + 4], out[8 * g + 5], out[8 * g + 6], out[8 * g + 7]));
}

// The merge of nsplit key splits: the load-batched kernel when the splits fit it, else the
// general one.
static void launch_attention_combine(hipStream_t s, const float *part, float *y, uint32_t rows, uint32_t hd,
                                     uint32_t nsplit, uint16_t *xs, uint32_t heads) {
  const bool fits = (uint64_t)nsplit * rows * (hd + 2) * 4 < (1ull << 31);
  if (fits && nsplit <= 4)
    hipLaunchKernelGGL(k_attention_combine_s<4>, dim3(rows), dim3(128), 0, s, part, y, rows, hd, nsplit, xs, heads);
  else if (fits && nsplit <= 8)
    hipLaunchKernelGGL(k_attention_combine_s<8>, dim3(rows), dim3(128), 0, s, part, y, rows, hd, nsplit, xs, heads);
  else if (fits && nsplit <= 16)
    hipLaunchKernelGGL(k_attention_combine_s<16>, dim3(rows), dim3(128), 0, s, part, y, rows, hd, nsplit, xs, heads);
  else
    hipLaunchKernelGGL(k_attention_combine, dim3(rows), dim3(128), 0, s, part, y, rows, hd, nsplit, xs, heads);
}

// Prompt batches on the f32 matrix cores (v_mfma_f32_16x16x4_f32: f32 products, f32 sums, as
// the f32 shader computes them). A wavefront owns 16 consecutive queries of one head; the
// four wavefronts of a workgroup share one kv head and stage 64-key tiles of K (row-major)
// and V (transposed) in LDS. Scores are formed transposed, S^T = K Q^T, so lane (g, c) holds
// keys 4g..4g+3 of query row c: a row's running max and sum live in its own lanes (two
// cross-lane steps per tile) and the probabilities already sit in the B-operand layout of
// O^T += V^T P^T. The k summation index of both products walks d (and keys) in the order
// 16t + 4g + u, which turns each operand fetch into one 16-byte LDS read per four MFMAs.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t AP_T = 64;  // keys per LDS tile

template <uint32_t HD>
constexpr size_t attn_prompt_lds() { return sizeof(float) * ((size_t)AP_T * (HD + 4) + (size_t)HD * (AP_T + 4)); }

template <uint32_t HD, class E>
__global__ __launch_bounds__(256) void k_attn_prompt(AttnK a) {
  constexpr uint32_t T = AP_T, KS = HD + 4, VS = T + 4, NT = HD / 16;
  extern __shared__ float lds[];
  float *Ks = lds, *Vt = lds + T * KS;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, c = lane & 15;
  const uint32_t kv = blockIdx.x, z = blockIdx.z, group = a.group;
  const uint32_t nqt = (a.batch + 15) / 16;
  const uint32_t ti = blockIdx.y * 4 + wv, qt = ti / group, h = kv * group + ti % group;
  const bool tile_ok = qt < nqt;
  const uint32_t s0 = a.start_dev ? (uint32_t)*a.start_dev : a.start;

  // Key range of the workgroup (its first and last query tiles), split into z chunks.
  const uint32_t qt_lo = blockIdx.y * 4 / group;
  const uint32_t qt_hi = min((blockIdx.y * 4 + 3) / group, nqt - 1);
  const uint32_t first_end = s0 + qt_lo * 16 + 1, last_end = s0 + min(a.batch, (qt_hi + 1) * 16);
  const uint32_t begin0 = first_end - min(first_end, a.window);
  uint32_t chunk = (last_end - begin0 + a.nsplit - 1) / a.nsplit;
  chunk = (chunk + T - 1) / T * T;
  const uint32_t lo = begin0 + z * chunk, hi = min(lo + chunk, last_end);

  // This lane's query row and the keys it sees; the wavefront's union of them.
  const uint32_t b = qt * 16 + c;
  const bool row_ok = tile_ok && b < a.batch;
  const uint32_t end_b = s0 + b + 1, begin_b = end_b - min(end_b, a.window);
  const uint32_t wq_end = s0 + (tile_ok ? min(a.batch, qt * 16 + 16) : 0);
  const uint32_t wq_first = s0 + qt * 16 + 1, wq_begin = wq_first - min(wq_first, a.window);

  f32x4 qr[NT], o[NT];
#pragma unroll
  for (uint32_t t = 0; t < NT; t++) {
    qr[t] = row_ok ? *(const f32x4 *)(a.q + ((uint64_t)b * a.heads + h) * HD + 16 * t + 4 * g) : f32x4{0, 0, 0, 0};
    o[t] = f32x4{0, 0, 0, 0};
  }
  float m = -INFINITY, l = 0.f;

  for (uint32_t t0 = lo; t0 < hi; t0 += T) {
    __syncthreads();
    for (uint32_t i = tid; i < T * HD / 4; i += 256) {
      const uint32_t j = i / (HD / 4), d = (i % (HD / 4)) * 4, t = t0 + j;
      f32x4 kk = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
      if (t < hi) {
        const uint64_t src = ((uint64_t)(t % a.capacity) * a.kvh + kv) * HD + d;
        const float4 k4 = kv_get4<E>(a.k, src), v4 = kv_get4<E>(a.v, src);
        kk = f32x4{k4.x, k4.y, k4.z, k4.w};
        vv = f32x4{v4.x, v4.y, v4.z, v4.w};
      }
      *(f32x4 *)(Ks + j * KS + d) = kk;
      Vt[(d + 0) * VS + j] = vv.x;
      Vt[(d + 1) * VS + j] = vv.y;
      Vt[(d + 2) * VS + j] = vv.z;
      Vt[(d + 3) * VS + j] = vv.w;
    }
    __syncthreads();
    const uint32_t k0 = max(t0, wq_begin), k1 = min(min(t0 + T, hi), wq_end);
    if (!tile_ok || k0 >= k1) continue;  // wavefront-uniform: none of its rows sees this tile
    float s[4][4];
    bool live[4];
#pragma unroll
    for (uint32_t kb = 0; kb < 4; kb++) {
      const uint32_t kt = t0 + kb * 16;
      live[kb] = kt < k1 && kt + 16 > k0;
      f32x4 acc = {0, 0, 0, 0};
      if (live[kb]) {
#pragma unroll
        for (uint32_t t = 0; t < NT; t++) {
          const f32x4 kf = *(const f32x4 *)(Ks + (kb * 16 + c) * KS + 16 * t + 4 * g);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.x, qr[t].x, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.y, qr[t].y, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.z, qr[t].z, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.w, qr[t].w, acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (uint32_t r = 0; r < 4; r++) {
        const uint32_t key = kt + 4 * g + r;
        s[kb][r] = (live[kb] && row_ok && key >= begin_b && key < end_b && key < hi) ? acc[r] * a.scale : -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t kb = 0; kb < 4; kb++)
#pragma unroll
      for (uint32_t r = 0; r < 4; r++) mx = fmaxf(mx, s[kb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    const float corr = mn == -INFINITY ? 1.f : expf(m - mn);
    float sum = 0.f;
#pragma unroll
    for (uint32_t kb = 0; kb < 4; kb++)
#pragma unroll
      for (uint32_t r = 0; r < 4; r++) {
        const float p = s[kb][r] == -INFINITY ? 0.f : expf(s[kb][r] - mn);
        s[kb][r] = p;
        sum += p;
      }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    l = l * corr + sum;
    m = mn;
#pragma unroll
    for (uint32_t t = 0; t < NT; t++) o[t] *= corr;
#pragma unroll
    for (uint32_t kb = 0; kb < 4; kb++) {
      if (!live[kb]) continue;
#pragma unroll
      for (uint32_t t = 0; t < NT; t++) {
        const f32x4 vf = *(const f32x4 *)(Vt + (t * 16 + c) * VS + kb * 16 + 4 * g);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.x, s[kb][0], o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.y, s[kb][1], o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.z, s[kb][2], o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.w, s[kb][3], o[t], 0, 0, 0);
      }
    }
  }
  if (!row_ok) return;
  // lane (g, c) holds O^T[16t + 4g + r][row c]
  const uint64_t row = (uint64_t)b * a.heads + h;
  if (a.nsplit == 1) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (uint32_t t = 0; t < NT; t++) *(f32x4 *)(a.y + row * HD + 16 * t + 4 * g) = o[t] * inv;
  } else {
    float *pp = a.part + ((uint64_t)z * a.batch * a.heads + row) * (HD + 2);
    if (g == 0) { pp[0] = m; pp[1] = l; }
#pragma unroll
    for (uint32_t t = 0; t < NT; t++)
#pragma unroll
      for (uint32_t r = 0; r < 4; r++) pp[2 + 16 * t + 4 * g + r] = o[t][r];
  }
}

template <uint32_t HD, class E>
static hipError_t launch_attn_prompt(hipStream_t s, AttnK a, const AttnArgs &in, uint32_t nsplit) {
  const uint32_t nqt = (in.batch + 15) / 16;
  a.nsplit = nsplit;
  constexpr size_t lds = attn_prompt_lds<HD>();
  if (lds > 65536) lds_opt_in((const void *)k_attn_prompt<HD, E>);
  hipLaunchKernelGGL((k_attn_prompt<HD, E>), dim3(in.kv_heads, (nqt * a.group + 3) / 4, nsplit), dim3(256), lds, s, a);
  WGD_HIP(hipGetLastError());
  if (nsplit > 1) {
    uint16_t *xs = in.xs && in.hd % 8 == 0 && in.heads * in.hd % 64 == 0 ? in.xs : nullptr;
    launch_attention_combine(s, (const float *)in.partial, in.y, in.batch * in.heads, in.hd, nsplit, xs, in.heads);
    WGD_HIP(hipGetLastError());
    if (in.xs_written) *in.xs_written = xs != nullptr;
  }
  return hipSuccess;
}

static uint32_t tile_keys(uint32_t hd) {
  uint32_t t = 4096 / hd;
  if (t > 64) t = 64;
  if (t < 1) t = 1;
  return t;
}

uint64_t attention_scratch_floats(uint32_t heads, uint32_t hd, uint32_t batch, uint32_t max_splits) {
  return (uint64_t)max_splits * batch * heads * (hd + 2);
}

// How a launch runs: the MFMA prompt kernel (hd 64/128/256 with 16-byte aligned operands) or
// the generic one (query blocks of qb tokens, tiles of T keys), and the number of key
// chunks: as many as fill the chip, fewer when `partial_floats` holds fewer partials.
struct AttnPlan { uint32_t mfma_hd, nsplit, qb, R, T, qblocks; };
static bool attn_plan(const AttnArgs &in, uint64_t partial_floats, AttnPlan &p) {
  const uint32_t group = in.heads / in.kv_heads;
  // Key range bound: the host start when known, else the whole ring/window.
  uint32_t keys = in.window;
  if (!in.start_dev) {
    uint32_t last_end = in.start + in.batch;
    uint32_t first_end = in.start + 1;
    uint32_t begin0 = first_end - (first_end < in.window ? first_end : in.window);
    keys = last_end - begin0;
  } else if (keys > in.capacity + in.batch) {
    keys = in.capacity + in.batch;
  }
  const bool aligned = ((uintptr_t)in.q | (uintptr_t)in.k | (uintptr_t)in.v | (uintptr_t)in.y) % 16 == 0;
  p = AttnPlan{};
  uint32_t tiles, want;
  if (aligned && (in.hd == 64 || in.hd == 128 || in.hd == 256)) {
    p.mfma_hd = in.hd;
    const uint32_t nqt = (in.batch + 15) / 16;
    const uint32_t wgs = in.kv_heads * ((nqt * group + 3) / 4);
    tiles = (keys + AP_T - 1) / AP_T;
    want = ((uint32_t)device_cu_count() * 2 + wgs - 1) / wgs;  // two workgroups per CU: a second wavefront per SIMD
  } else {
    p.qb = group >= 16 ? 1 : 16 / group;
    if (p.qb > in.batch) p.qb = in.batch;
    p.R = p.qb * group;
    if (p.R > 16) return false;
    p.T = tile_keys(in.hd);
    p.qblocks = (in.batch + p.qb - 1) / p.qb;
    tiles = (keys + p.T - 1) / p.T;
    want = (uint32_t)device_cu_count() * 4 / (in.kv_heads * p.qblocks);
  }
  uint32_t nsplit = tiles < want ? tiles : want;
  if (nsplit < 1) nsplit = 1;
  if (nsplit > 1) {
    const uint64_t per_split = (uint64_t)in.batch * in.heads * (in.hd + 2);
    const uint64_t fit = partial_floats / per_split;
    if (fit < nsplit) nsplit = fit > 1 ? (uint32_t)fit : 1;
  }
  p.nsplit = nsplit;
  return true;
}

uint64_t attention_partial_need(const AttnArgs &in) {
  AttnPlan p;
  if (!in.batch || !in.kv_heads || in.heads % in.kv_heads || !attn_plan(in, UINT64_MAX, p) || p.nsplit < 2) return 0;
  return (uint64_t)p.nsplit * in.batch * in.heads * (in.hd + 2);
}

hipError_t attention(hipStream_t s, const AttnArgs &in) {
  if (!in.batch) return hipSuccess;
  if (!in.kv_heads || in.heads % in.kv_heads || in.hd == 0 || in.hd > 512 || !in.capacity || !in.window)
    return hipErrorInvalidValue;
  AttnK a;
  a.q = in.q; a.k = in.k; a.v = in.v; a.y = in.y; a.part = in.partial;
  a.heads = in.heads; a.kvh = in.kv_heads; a.hd = in.hd; a.start = in.start; a.start_dev = in.start_dev;
  a.scale = in.scale; a.window = in.window; a.capacity = in.capacity; a.batch = in.batch;
  a.group = in.heads / in.kv_heads;
  AttnPlan p;
  if (!attn_plan(in, in.partial ? in.partial_floats : 0, p)) return hipErrorInvalidValue;
  if (p.mfma_hd == 64) return in.kv16 ? launch_attn_prompt<64, _Float16>(s, a, in, p.nsplit) : launch_attn_prompt<64, float>(s, a, in, p.nsplit);
  if (p.mfma_hd == 128) return in.kv16 ? launch_attn_prompt<128, _Float16>(s, a, in, p.nsplit) : launch_attn_prompt<128, float>(s, a, in, p.nsplit);
  if (p.mfma_hd == 256) return in.kv16 ? launch_attn_prompt<256, _Float16>(s, a, in, p.nsplit) : launch_attn_prompt<256, float>(s, a, in, p.nsplit);
  a.qb = p.qb; a.R = p.R; a.T = p.T;
  const uint32_t qblocks = p.qblocks, nsplit = p.nsplit;
  a.nsplit = nsplit;
  size_t lds = sizeof(float) * ((size_t)a.T * (in.hd + 1) + (size_t)a.T * in.hd + (size_t)a.R * in.hd +
                                (size_t)a.R * a.T + 3 * a.R);
  if (in.kv16) {
    if (lds > 65536) lds_opt_in((const void *)k_attention<_Float16>);
    hipLaunchKernelGGL(k_attention<_Float16>, dim3(in.kv_heads, qblocks, nsplit), dim3(256), lds, s, a);
  } else {
    if (lds > 65536) lds_opt_in((const void *)k_attention<float>);
    hipLaunchKernelGGL(k_attention<float>, dim3(in.kv_heads, qblocks, nsplit), dim3(256), lds, s, a);
  }
  WGD_HIP(hipGetLastError());
  if (nsplit > 1) {
    launch_attention_combine(s, (const float *)in.partial, in.y, in.batch * in.heads, in.hd, nsplit, nullptr, in.heads);
    WGD_HIP(hipGetLastError());
  }
  return hipSuccess;
}

// ------------------------------------------------------------------ decode step
//
// One token: a workgroup per (kv head, chunk of 32 * NB keys), four wavefronts of KPB-key
// batches. The prologue normalises and rotates the group's query heads and the new key
// (angles in f64 as in k_rope) into LDS; the workgroup whose chunk holds the current
// position writes the new key and value into the ring (the slot of the position,
// pos % capacity: the ring keeps at least the window, so no other chunk of this launch
// reads it) and uses the fresh values for that key. Lanes span the head dimension (EL
// floats each): a key row is one coalesced load, each score a DPP wave sum broadcast as a
// scalar, and the online softmax state (m, l) is uniform per wavefront. The four
// wavefronts merge through LDS and the workgroup leaves (max, sum, unnormalised output)
// per query head; k_attn_comb merges the chunks.
constexpr uint32_t AD_KPB = 8;   // keys per wavefront batch
constexpr uint32_t AD_WAVES = 4;

struct AttnDecK {
  const float *q, *k, *v; void *kc, *vc; const float *qn, *kn; float *part;  // kc, vc: ring of E elements
  const int32_t *pos;
  const float *cs;   // this token's rotation: cos of pair i at [i], sin at [rot / 2 + i]
  uint32_t heads, kvh, rot, cap, window, group, chunk, nsplit;
  float scale, eps; int mode;
};

// Chunk epilogue of both decode kernels: merge the four wavefronts' (max, sum, output) into
// the chunk's partial, which k_attn_comb merges with the other chunks of the head.
template <int G, uint32_t HD>
__device__ __forceinline__ void chunk_epilogue(const AttnDecK &a, uint32_t kv, uint32_t z, const float (*wm)[G],
                                               const float (*wl)[G], const float (*wo)[G][HD]) {
  const uint32_t g = a.group;
  for (uint32_t j = threadIdx.x; j < g * HD; j += blockDim.x) {
    const uint32_t i = j / HD, d = j % HD;
    float M = -INFINITY;
#pragma unroll
    for (uint32_t u = 0; u < AD_WAVES; u++) M = fmaxf(M, wm[u][i]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < AD_WAVES; u++) {
      if (wm[u][i] == -INFINITY) continue;
      const float f = expf(wm[u][i] - M);
      L += wl[u][i] * f;
      O += wo[u][i][d] * f;
    }
    float *pp = a.part + (((uint64_t)kv * g + i) * a.nsplit + z) * (HD + 2);
    if (d == 0) { pp[0] = M; pp[1] = L; }
    pp[2 + d] = O;
  }
}

template <int EL, int G, class E>
__global__ __launch_bounds__(256) void k_attn_dec(AttnDecK a) {
  constexpr uint32_t HD = 64 * EL;
  __shared__ float vec[(G + 1) * HD];        // query heads, then the new key
  __shared__ float csn[HD];                   // cos / sin per rotation pair
  __shared__ float wm[AD_WAVES][G], wl[AD_WAVES][G];
  __shared__ float wo[AD_WAVES][G][HD];
  const uint32_t lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t kv = blockIdx.x, z = blockIdx.y, g = a.group;
  const uint32_t pos = (uint32_t)__builtin_amdgcn_readfirstlane(*a.pos);
  const uint32_t end = pos + 1, win = end < a.window ? end : a.window, begin = end - win;
  const uint32_t lo = begin + z * a.chunk;
  if (lo >= end) return;
  const uint32_t hi = lo + a.chunk < end ? lo + a.chunk : end;
  const uint32_t nb = a.chunk / (AD_WAVES * AD_KPB);
  const uint64_t rowf = (uint64_t)a.kvh * HD;  // floats per ring slot
  // ---- key batch loads (rows past the chunk re-read its first key; they are masked)
  float kr[AD_KPB][EL], vr[AD_KPB][EL];
  auto load_batch = [&](uint32_t b) {
#pragma unroll
    for (uint32_t k = 0; k < AD_KPB; k++) {
      uint32_t t = lo + (b * AD_WAVES + w) * AD_KPB + k;
      if (t >= hi) t = lo;
      const uint64_t base = (uint64_t)(t % a.cap) * rowf + (uint64_t)kv * HD + lane * EL;
#pragma unroll
      for (int e = 0; e < EL; e++) { kr[k][e] = kv_get<E>(a.kc, base + e); vr[k][e] = kv_get<E>(a.vc, base + e); }
    }
  };
  load_batch(0);
  // ---- prologue: Q/K norm and RoPE of the group's query heads and the new key
  const uint32_t half = a.rot / 2;
  for (uint32_t i = threadIdx.x; i < half; i += blockDim.x) {
    csn[2 * i] = a.cs[i];
    csn[2 * i + 1] = a.cs[half + i];
  }
  for (uint32_t it = w; it <= g; it += AD_WAVES) {
    const bool isk = it == g;
    const float *src = isk ? a.k + (uint64_t)kv * HD : a.q + ((uint64_t)kv * g + it) * HD;
    float x[EL];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EL; e++) { x[e] = src[lane * EL + e]; ss += x[e] * x[e]; }
    if (a.mode == 0) {
      const float inv = 1.f / sqrtf(wave_total(ss) / (float)HD + a.eps);
      const float *wn = isk ? a.kn : a.qn;
#pragma unroll
      for (int e = 0; e < EL; e++) x[e] = x[e] * wn[lane * EL + e] * inv;
    }
#pragma unroll
    for (int e = 0; e < EL; e++) vec[it * HD + lane * EL + e] = x[e];
  }
  __syncthreads();
  for (uint32_t j = threadIdx.x; j < (g + 1) * half; j += blockDim.x) {
    const uint32_t it = j / half, i = j % half;
    const uint32_t ia = a.mode == 2 ? 2 * i : i, ib = a.mode == 2 ? 2 * i + 1 : i + half;
    float *v = vec + it * HD;
    const float c = csn[2 * i], sn = csn[2 * i + 1], xa = v[ia], xb = v[ib];
    v[ia] = xa * c - xb * sn;
    v[ib] = xa * sn + xb * c;
  }
  __syncthreads();
  const bool mine = pos >= lo && pos < hi;
  if (mine) {
    const uint64_t slot = (uint64_t)(pos % a.cap) * rowf + (uint64_t)kv * HD;
    for (uint32_t d = threadIdx.x; d < HD; d += blockDim.x) {
      kv_put(a.kc, slot + d, vec[g * HD + d], sizeof(E) == 2);
      kv_put(a.vc, slot + d, a.v[(uint64_t)kv * HD + d], sizeof(E) == 2);
    }
  }
  float qr[G][EL], kf[EL], vf[EL];
#pragma unroll
  for (int i = 0; i < G; i++)
#pragma unroll
    for (int e = 0; e < EL; e++) qr[i][e] = (uint32_t)i < g ? vec[i * HD + lane * EL + e] : 0.f;
#pragma unroll
  for (int e = 0; e < EL; e++) {
    kf[e] = (float)(E)vec[g * HD + lane * EL + e];
    vf[e] = (float)(E)a.v[(uint64_t)kv * HD + lane * EL + e];
  }
  // ---- keys
  float m[G], l[G], o[G][EL];
#pragma unroll
  for (int i = 0; i < G; i++) {
    m[i] = -INFINITY; l[i] = 0.f;
#pragma unroll
    for (int e = 0; e < EL; e++) o[i][e] = 0.f;
  }
  for (uint32_t b = 0; b < nb; b++) {
    if (b > 0) load_batch(b);
    const uint32_t t0 = lo + (b * AD_WAVES + w) * AD_KPB;
    if (t0 >= hi) break;  // uniform: later batches of this wavefront are past the chunk too
    float sc[AD_KPB][G];
#pragma unroll
    for (uint32_t k = 0; k < AD_KPB; k++) {
      const bool fresh = t0 + k == pos;
#pragma unroll
      for (int e = 0; e < EL; e++) {
        if (fresh) { kr[k][e] = kf[e]; vr[k][e] = vf[e]; }
      }
#pragma unroll
      for (int i = 0; i < G; i++) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < EL; e++) d += qr[i][e] * kr[k][e];
        sc[k][i] = t0 + k < hi ? wave_total(d) * a.scale : -INFINITY;
      }
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
      float bm = sc[0][i];
#pragma unroll
      for (uint32_t k = 1; k < AD_KPB; k++) bm = fmaxf(bm, sc[k][i]);
      const float mn = fmaxf(m[i], bm);  // finite: key t0 is inside the chunk
      const float corr = m[i] == -INFINITY ? 0.f : expf(m[i] - mn);
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < EL; e++) o[i][e] *= corr;
#pragma unroll
      for (uint32_t k = 0; k < AD_KPB; k++) {
        const float p = sc[k][i] == -INFINITY ? 0.f : expf(sc[k][i] - mn);
        ps += p;
#pragma unroll
        for (int e = 0; e < EL; e++) o[i][e] += p * vr[k][e];
      }
      l[i] = l[i] * corr + ps;
      m[i] = mn;
    }
  }
  // ---- merge the wavefronts, then the chunks
#pragma unroll
  for (int i = 0; i < G; i++) {
    if (lane == 0) { wm[w][i] = m[i]; wl[w][i] = l[i]; }
#pragma unroll
    for (int e = 0; e < EL; e++) wo[w][i][lane * EL + e] = o[i][e];
  }
  __syncthreads();
  chunk_epilogue<G, HD>(a, kv, z, wm, wl, wo);
}

// ------------------------------------------------------------------ decode step, 16-byte lanes
//
// One token: a workgroup per (kv head, chunk of keys), four wavefronts. A lane holds 8
// elements of a key row (two 16-byte pieces, elements 4s..4s+3 and HD/2 + 4s..+3 for lane
// s of the key's LPK = HD/8 lanes), so one wavefront load instruction covers KPW = 64/LPK
// whole key rows, and a score needs a log2(LPK)-step DPP sum over the key's lanes rather
// than a wave-wide one. Each key slot (a group of LPK lanes) keeps its own online-softmax
// state over the keys it visits; the slots of a wavefront merge once at the end, then the
// wavefronts through LDS. A wavefront loads AD2_DB key iterations at once. The prologue
// normalises and rotates the group's query heads and the new key in registers (angles in
// f64 as in k_rope); the workgroup whose chunk holds the position writes the new key and
// value into the ring (slot pos % capacity: the ring keeps at least the window, so no
// other chunk of this launch reads it) and uses the fresh values for that key.
constexpr uint32_t AD2_DB = 2;  // key iterations (KPW keys each) per wavefront load batch

template <uint32_t LPK>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_mov<0xB1>(v);                       // quad xor 1
  v += dpp_mov<0x4E>(v);                       // quad xor 2
  if (LPK >= 8) v += dpp_mov<0x141>(v);        // half-row mirror: the other quad of 8
  if (LPK >= 16) v += dpp_mov<0x140>(v);       // row mirror: the other 8 of 16
  if (LPK >= 32) v += __shfl_xor(v, 16, 64);   // the other row of 32
  return v;
}

// Sum / max over the key slots of a wavefront (lanes that differ in the bits above LPK),
// left in every lane: DPP row rotation by 8 (slots of 8 lanes), then gfx950's row swaps
// (v_permlane16_swap pairs rows 0-1 and 2-3, v_permlane32_swap the two halves), all VALU.
template <uint32_t LPK, bool MAX>
__device__ __forceinline__ float slots_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  if (LPK <= 8) v = op(v, dpp_mov<0x128>(v));  // row_ror:8 = lane xor 8 within a row
  if (LPK <= 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <uint32_t HD, int G, bool ADJ, class E>
__global__ __launch_bounds__(256) void k_attn_dec2(AttnDecK a) {
  constexpr uint32_t LPK = HD / 8, KPW = 64 / LPK, NW = AD_WAVES;
  __shared__ float wm[AD_WAVES][G], wl[AD_WAVES][G];
  __shared__ float wo[AD_WAVES][G][HD];
  const uint32_t lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t kv = blockIdx.x, z = blockIdx.y, g = a.group;
  const uint32_t slot = lane / LPK, sub = lane % LPK;
  const uint32_t e0 = 4 * sub, e1 = HD / 2 + 4 * sub;  // this lane's two 4-element pieces
  // ---- loads that do not depend on the position
  float4 q[G][2], kn[2], vn[2], qw[2], kw[2];
#pragma unroll
  for (int i = 0; i < G; i++) {
    const float *qs = a.q + ((uint64_t)kv * g + ((uint32_t)i < g ? i : 0)) * HD;
    q[i][0] = *(const float4 *)(qs + e0);
    q[i][1] = *(const float4 *)(qs + e1);
  }
  kn[0] = *(const float4 *)(a.k + (uint64_t)kv * HD + e0);
  kn[1] = *(const float4 *)(a.k + (uint64_t)kv * HD + e1);
  vn[0] = *(const float4 *)(a.v + (uint64_t)kv * HD + e0);
  vn[1] = *(const float4 *)(a.v + (uint64_t)kv * HD + e1);
  if (a.mode == 0) {
    qw[0] = *(const float4 *)(a.qn + e0); qw[1] = *(const float4 *)(a.qn + e1);
    kw[0] = *(const float4 *)(a.kn + e0); kw[1] = *(const float4 *)(a.kn + e1);
  }
  // rotation of this lane's pairs: adjacent pairs (e, e+1) inside a piece, or half-split
  // pairs (e0 + c, e1 + c) across the two pieces
  float cr[4], sr[4];
  const uint32_t half = a.rot / 2;
  if (ADJ) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t pi = (c < 2 ? e0 : e1) / 2 + (c & 1);
      cr[c] = a.cs[pi]; sr[c] = a.cs[half + pi];
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; c++) { cr[c] = a.cs[e0 + c]; sr[c] = a.cs[half + e0 + c]; }
  }
  const uint32_t pos = (uint32_t)__builtin_amdgcn_readfirstlane(*a.pos);
  const uint32_t end = pos + 1, win = end < a.window ? end : a.window, begin = end - win;
  const uint32_t lo = begin + z * a.chunk;
  if (lo >= end) return;
  const uint32_t hi = lo + a.chunk < end ? lo + a.chunk : end;
  const uint64_t rowf = (uint64_t)a.kvh * HD;
  // ---- the first batch of keys goes out before the norm and rotation arithmetic
  float4 kb[AD2_DB][2], vb[AD2_DB][2];
  auto key_of = [&](uint32_t b, uint32_t d) { return lo + ((b * AD2_DB + d) * NW + w) * KPW + slot; };
  auto load_batch = [&](uint32_t b) {
#pragma unroll
    for (uint32_t d = 0; d < AD2_DB; d++) {
      uint32_t t = key_of(b, d);
      if (t >= hi) t = lo;  // masked below; any valid row
      const uint64_t r = (uint64_t)(t % a.cap) * rowf + (uint64_t)kv * HD;
      kb[d][0] = kv_get4<E>(a.kc, r + e0); kb[d][1] = kv_get4<E>(a.kc, r + e1);
      vb[d][0] = kv_get4<E>(a.vc, r + e0); vb[d][1] = kv_get4<E>(a.vc, r + e1);
    }
  };
  load_batch(0);
  // ---- Q/K RMSNorm (mode 0) and rotation, in registers
  auto sq4 = [](const float4 &v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; };
  auto mul4 = [](const float4 &v, const float4 &u, float f) { return make_float4(v.x * u.x * f, v.y * u.y * f, v.z * u.z * f, v.w * u.w * f); };
  if (a.mode == 0) {
#pragma unroll
    for (int i = 0; i < G; i++) {
      const float inv = 1.f / sqrtf(group_sum<LPK>(sq4(q[i][0]) + sq4(q[i][1])) / (float)HD + a.eps);
      q[i][0] = mul4(q[i][0], qw[0], inv); q[i][1] = mul4(q[i][1], qw[1], inv);
    }
    const float inv = 1.f / sqrtf(group_sum<LPK>(sq4(kn[0]) + sq4(kn[1])) / (float)HD + a.eps);
    kn[0] = mul4(kn[0], kw[0], inv); kn[1] = mul4(kn[1], kw[1], inv);
  }
  auto rot = [&](float4 (&v)[2]) {
    if (ADJ) {
      // pairs (x, y) and (z, w) of each piece: rotation slots 0, 1 (piece 0) and 2, 3 (piece 1)
      float x, y;
      x = v[0].x; y = v[0].y; v[0].x = x * cr[0] - y * sr[0]; v[0].y = x * sr[0] + y * cr[0];
      x = v[0].z; y = v[0].w; v[0].z = x * cr[1] - y * sr[1]; v[0].w = x * sr[1] + y * cr[1];
      x = v[1].x; y = v[1].y; v[1].x = x * cr[2] - y * sr[2]; v[1].y = x * sr[2] + y * cr[2];
      x = v[1].z; y = v[1].w; v[1].z = x * cr[3] - y * sr[3]; v[1].w = x * sr[3] + y * cr[3];
    } else {
      float *p0 = &v[0].x, *p1 = &v[1].x;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float xa = p0[c], xb = p1[c];
        p0[c] = xa * cr[c] - xb * sr[c];
        p1[c] = xa * sr[c] + xb * cr[c];
      }
    }
  };
#pragma unroll
  for (int i = 0; i < G; i++) rot(q[i]);
  rot(kn);
  if (sizeof(E) == 2) {
    // the new key and value as the f16 ring holds them, so every chunk sees the same values
    auto rnd = [](float4 &v) { v = make_float4((float)(E)v.x, (float)(E)v.y, (float)(E)v.z, (float)(E)v.w); };
    rnd(kn[0]); rnd(kn[1]); rnd(vn[0]); rnd(vn[1]);
  }
  if (pos >= lo && pos < hi && w == 0 && slot == 0) {
    const uint64_t r = (uint64_t)(pos % a.cap) * rowf + (uint64_t)kv * HD;
    kv_put4<E>(a.kc, r + e0, kn[0]); kv_put4<E>(a.kc, r + e1, kn[1]);
    kv_put4<E>(a.vc, r + e0, vn[0]); kv_put4<E>(a.vc, r + e1, vn[1]);
  }
  // ---- keys
  float m[G], l[G];
  float4 o[G][2];
#pragma unroll
  for (int i = 0; i < G; i++) { m[i] = -INFINITY; l[i] = 0.f; o[i][0] = o[i][1] = make_float4(0.f, 0.f, 0.f, 0.f); }
  const uint32_t nb = (a.chunk + AD2_DB * NW * KPW - 1) / (AD2_DB * NW * KPW);
  auto dot8 = [](const float4 (&x)[2], const float4 (&y)[2]) {
    float s = x[0].x * y[0].x;
    s = fmaf(x[0].y, y[0].y, s); s = fmaf(x[0].z, y[0].z, s); s = fmaf(x[0].w, y[0].w, s);
    s = fmaf(x[1].x, y[1].x, s); s = fmaf(x[1].y, y[1].y, s); s = fmaf(x[1].z, y[1].z, s);
    return fmaf(x[1].w, y[1].w, s);
  };
  for (uint32_t b = 0; b < nb; b++) {
    if (lo + (b * AD2_DB * NW + w) * KPW >= hi) break;  // uniform: this wavefront's keys are all past the chunk
    if (b > 0) load_batch(b);
    float sc[AD2_DB][G];
#pragma unroll
    for (uint32_t d = 0; d < AD2_DB; d++) {
      const uint32_t t = key_of(b, d);
      if (t == pos) { kb[d][0] = kn[0]; kb[d][1] = kn[1]; vb[d][0] = vn[0]; vb[d][1] = vn[1]; }
#pragma unroll
      for (int i = 0; i < G; i++) {
        const float s = group_sum<LPK>(dot8(q[i], kb[d])) * a.scale;
        sc[d][i] = t < hi ? s : -INFINITY;
      }
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
      float bm = sc[0][i];
#pragma unroll
      for (uint32_t d = 1; d < AD2_DB; d++) bm = fmaxf(bm, sc[d][i]);
      const float mn = fmaxf(m[i], bm);
      const float corr = m[i] == -INFINITY ? 0.f : expf(m[i] - mn);
      float ps = 0.f;
      float4 o0 = make_float4(o[i][0].x * corr, o[i][0].y * corr, o[i][0].z * corr, o[i][0].w * corr);
      float4 o1 = make_float4(o[i][1].x * corr, o[i][1].y * corr, o[i][1].z * corr, o[i][1].w * corr);
#pragma unroll
      for (uint32_t d = 0; d < AD2_DB; d++) {
        const float p = sc[d][i] == -INFINITY ? 0.f : expf(sc[d][i] - mn);
        ps += p;
        o0.x = fmaf(p, vb[d][0].x, o0.x); o0.y = fmaf(p, vb[d][0].y, o0.y); o0.z = fmaf(p, vb[d][0].z, o0.z); o0.w = fmaf(p, vb[d][0].w, o0.w);
        o1.x = fmaf(p, vb[d][1].x, o1.x); o1.y = fmaf(p, vb[d][1].y, o1.y); o1.z = fmaf(p, vb[d][1].z, o1.z); o1.w = fmaf(p, vb[d][1].w, o1.w);
      }
      o[i][0] = o0; o[i][1] = o1;
      l[i] = l[i] * corr + ps;
      m[i] = mn;
    }
  }
  // ---- merge the wavefront's key slots (lanes slot * LPK + sub), then the wavefronts
#pragma unroll
  for (int i = 0; i < G; i++) {
    const float M = slots_reduce<LPK, true>(m[i]);
    const float f = m[i] == -INFINITY ? 0.f : expf(m[i] - M);
    const float L = slots_reduce<LPK, false>(l[i] * f);
    float v8[8] = {o[i][0].x * f, o[i][0].y * f, o[i][0].z * f, o[i][0].w * f, o[i][1].x * f, o[i][1].y * f, o[i][1].z * f, o[i][1].w * f};
#pragma unroll
    for (int c = 0; c < 8; c++) v8[c] = slots_reduce<LPK, false>(v8[c]);
    if (lane == 0) { wm[w][i] = M; wl[w][i] = L; }
    if (slot == 0) {
#pragma unroll
      for (int c = 0; c < 4; c++) { wo[w][i][e0 + c] = v8[c]; wo[w][i][e1 + c] = v8[4 + c]; }
    }
  }
  __syncthreads();
  // the wavefronts' rescaling factors once per head, then the chunk's partial
  __shared__ float wf[AD_WAVES][G], hM[G], hL[G];
  if (threadIdx.x < (uint32_t)G) {
    const uint32_t i = threadIdx.x;
    float M = -INFINITY;
#pragma unroll
    for (uint32_t u = 0; u < AD_WAVES; u++) M = fmaxf(M, wm[u][i]);
    float L = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < AD_WAVES; u++) {
      const float f = wm[u][i] == -INFINITY ? 0.f : expf(wm[u][i] - M);
      wf[u][i] = f;
      L += wl[u][i] * f;
    }
    hM[i] = M; hL[i] = L;
  }
  __syncthreads();
  for (uint32_t j = threadIdx.x; j < g * HD; j += blockDim.x) {
    const uint32_t i = j / HD, d = j % HD;
    float O = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < AD_WAVES; u++) O = fmaf(wo[u][i][d], wf[u][i], O);
    float *pp = a.part + (((uint64_t)kv * g + i) * a.nsplit + z) * (HD + 2);
    if (d == 0) { pp[0] = hM[i]; pp[1] = hL[i]; }
    pp[2 + d] = O;
  }
}

// Merge of the chunks of one query head: thread d owns output element d. The partials were
// written by the previous launch. Every load goes out at once, before the
// position arrives: raw buffer loads over the head's nsplit partials (zero past them), the
// first AD_ZB chunks' outputs in registers; chunks at or past the active count are masked
// afterwards. So the merge is one round trip.
constexpr uint32_t AD_MAX_SPLITS = 1024, AD_ZB = 32;
//
// With group > 0 (kv heads a multiple of 8) workgroup w, dispatched to XCD w % 8, merges a
// head of a kv head kv with kv % 8 == w % 8: the chunk launch's workgroup z * kv_heads + kv
// wrote that head's partials on the same XCD.
__global__ __launch_bounds__(256) void k_attn_comb(const float *part, float *y, QXOut qx, const int32_t *pos_dev,
                                                   uint32_t window, uint32_t chunk, uint32_t nsplit, uint32_t hd,
                                                   uint32_t group) {
  __shared__ float wz[AD_MAX_SPLITS];
  __shared__ float red[8];
  const uint32_t w = blockIdx.x, j = w / 8;
  const uint32_t h = group ? (w % 8 + 8 * (j / group)) * group + j % group : w;
  const uint32_t d = threadIdx.x, lane = d & 63, wv = d >> 6, nw = (blockDim.x + 63) >> 6;
  const uint32_t stride = hd + 2;
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(part + (uint64_t)h * nsplit * stride), 0, (int)(nsplit * stride * 4), 0x00020000);
  auto ld = [&](uint32_t idx) { return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, 4 * idx, 0, 0)); };
  float ov[AD_ZB];
#pragma unroll
  for (uint32_t k = 0; k < AD_ZB; k++) ov[k] = ld(k * stride + 2 + (d < hd ? d : 0));
  const float mz0 = ld(d * stride), lz0 = ld(d * stride + 1);
  const uint32_t pos = (uint32_t)__builtin_amdgcn_readfirstlane(*pos_dev);
  const uint32_t end = pos + 1, win = end < window ? end : window;
  const uint32_t nact = (win + chunk - 1) / chunk;
  float mz = d < nact ? mz0 : -INFINITY;
  for (uint32_t zz = d + blockDim.x; zz < nact; zz += blockDim.x) mz = fmaxf(mz, ld(zz * stride));
  float M = mz;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  if (lane == 0) red[wv] = M;
  __syncthreads();
  M = red[0];
  for (uint32_t u = 1; u < nw; u++) M = fmaxf(M, red[u]);
  float L = 0.f;
  if (d < nact) { const float f = expf(mz0 - M); wz[d] = f; L = lz0 * f; }
  for (uint32_t zz = d + blockDim.x; zz < nact; zz += blockDim.x) {
    const float f = expf(ld(zz * stride) - M);
    wz[zz] = f;
    L += ld(zz * stride + 1) * f;
  }
  L = wave_sum(L);
  __syncthreads();
  if (lane == 0) red[wv] = L;
  __syncthreads();
  L = 0.f;
  for (uint32_t u = 0; u < nw; u++) L += red[u];
  float O = 0.f;
#pragma unroll
  for (uint32_t k = 0; k < AD_ZB; k++) if (k < nact) O += ov[k] * wz[k];
  if (d < hd)
    for (uint32_t k = AD_ZB; k < nact; k++) O += ld(k * stride + 2 + d) * wz[k];
  const float out = O / L;
  if (d < hd) y[(uint64_t)h * hd + d] = out;
  if (qx.d0) qx_store(qx, h * hd + d, out, out, d < hd);
}

__global__ void k_inv_freq(double *f, uint32_t half, uint32_t rot, float theta) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < half; i += gridDim.x * blockDim.x)
    f[i] = pow((double)theta, -(double)(2 * i) / (double)rot);
}

hipError_t rope_inv_freq(hipStream_t s, double *f, uint32_t rot, float theta) {
  if (rot < 2 || rot % 2) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_inv_freq, dim3((rot / 2 + 255) / 256), dim3(256), 0, s, f, rot / 2, rot, theta);
  return hipGetLastError();
}

static uint32_t dec2_chunk(uint32_t capacity, uint32_t kvh, uint32_t hd);
static uint32_t dec_chunk(uint32_t capacity, uint32_t kvh) {
  // enough workgroups to cover the chip twice at full context, at most 512 keys each
  uint32_t nb = capacity * kvh / (AD_WAVES * AD_KPB * 2 * (uint32_t)device_cu_count());
  if (nb < 1) nb = 1;
  if (nb > 16) nb = 16;
  return nb * AD_WAVES * AD_KPB;
}

bool decode_attention_supported(uint32_t heads, uint32_t kv_heads, uint32_t hd) {
  return (hd == 64 || hd == 128 || hd == 256) && kv_heads && heads % kv_heads == 0 && heads / kv_heads <= 8;
}

// Partials of either decode kernel (the full-rotation one chunks by dec2_chunk, the other
// by dec_chunk).
uint64_t decode_attention_scratch_floats(uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t capacity) {
  const uint32_t c1 = dec_chunk(capacity, kv_heads), c2 = dec2_chunk(capacity, kv_heads, hd);
  const uint32_t n1 = (capacity + c1 - 1) / c1, n2 = (capacity + c2 - 1) / c2;
  return (uint64_t)heads * (n1 > n2 ? n1 : n2) * (hd + 2);
}

// Keys per workgroup of k_attn_dec2: whole load batches (AD2_DB * 4 wavefronts * KPW keys),
// enough workgroups to cover the chip twice over the ring, at most AD_MAX_SPLITS chunks.
static uint32_t dec2_chunk(uint32_t capacity, uint32_t kvh, uint32_t hd) {
  const uint32_t batch = AD2_DB * AD_WAVES * (64 / (hd / 8));
  uint32_t c = (uint32_t)(((uint64_t)capacity * kvh + 2 * device_cu_count() - 1) / (2 * device_cu_count()));
  c = (c + batch - 1) / batch * batch;
  if (c < batch) c = batch;
  while ((capacity + c - 1) / c > AD_MAX_SPLITS) c += batch;
  return c;
}

template <int EL, class E>
static void launch_dec(hipStream_t s, const AttnDecK &k, dim3 grid) {
  if (k.group <= 1) hipLaunchKernelGGL((k_attn_dec<EL, 1, E>), grid, dim3(256), 0, s, k);
  else if (k.group <= 2) hipLaunchKernelGGL((k_attn_dec<EL, 2, E>), grid, dim3(256), 0, s, k);
  else if (k.group <= 4) hipLaunchKernelGGL((k_attn_dec<EL, 4, E>), grid, dim3(256), 0, s, k);
  else hipLaunchKernelGGL((k_attn_dec<EL, 8, E>), grid, dim3(256), 0, s, k);
}
template <int EL>
static void launch_dec(hipStream_t s, const AttnDecK &k, dim3 grid, bool kv16) {
  kv16 ? launch_dec<EL, _Float16>(s, k, grid) : launch_dec<EL, float>(s, k, grid);
}

template <uint32_t HD, bool ADJ, class E>
static void launch_dec2(hipStream_t s, const AttnDecK &k, dim3 grid) {
  if (k.group <= 1) hipLaunchKernelGGL((k_attn_dec2<HD, 1, ADJ, E>), grid, dim3(256), 0, s, k);
  else if (k.group <= 2) hipLaunchKernelGGL((k_attn_dec2<HD, 2, ADJ, E>), grid, dim3(256), 0, s, k);
  else if (k.group <= 4) hipLaunchKernelGGL((k_attn_dec2<HD, 4, ADJ, E>), grid, dim3(256), 0, s, k);
  else hipLaunchKernelGGL((k_attn_dec2<HD, 8, ADJ, E>), grid, dim3(256), 0, s, k);
}
template <uint32_t HD>
static void launch_dec2(hipStream_t s, const AttnDecK &k, dim3 grid, bool adj, bool kv16) {
  if (kv16) adj ? launch_dec2<HD, true, _Float16>(s, k, grid) : launch_dec2<HD, false, _Float16>(s, k, grid);
  else adj ? launch_dec2<HD, true, float>(s, k, grid) : launch_dec2<HD, false, float>(s, k, grid);
}

hipError_t decode_attention(hipStream_t s, const DecodeAttnArgs &in) {
  if (!decode_attention_supported(in.heads, in.kv_heads, in.hd) || !in.capacity || !in.window || !in.pos ||
      !in.partial || !in.rope || !in.y || (in.mode == 0 && (!in.q_norm || !in.k_norm)) || in.rot > in.hd || in.rot % 2)
    return hipErrorInvalidValue;
  AttnDecK k;
  k.q = in.q; k.k = in.k; k.v = in.v; k.kc = in.kc; k.vc = in.vc; k.qn = in.q_norm; k.kn = in.k_norm;
  k.part = in.partial; k.pos = in.pos; k.cs = in.rope;
  k.heads = in.heads; k.kvh = in.kv_heads; k.rot = in.rot ? in.rot : in.hd; k.cap = in.capacity;
  k.window = in.window; k.group = in.heads / in.kv_heads;
  // full-width rotation runs the 16-byte-lane kernel, partial rotation the generic one
  const bool full = k.rot == in.hd;
  k.chunk = full ? dec2_chunk(in.capacity, in.kv_heads, in.hd) : dec_chunk(in.capacity, in.kv_heads);
  const uint32_t keys = in.window < in.capacity ? in.window : in.capacity;
  k.nsplit = (keys + k.chunk - 1) / k.chunk;
  if (k.nsplit > AD_MAX_SPLITS) return hipErrorInvalidValue;
  k.scale = in.scale; k.eps = in.eps; k.mode = in.mode;
  const dim3 grid(in.kv_heads, k.nsplit);
  if (full) {
    const bool adj = in.mode == 2;
    if (in.hd == 64) launch_dec2<64>(s, k, grid, adj, in.kv16);
    else if (in.hd == 128) launch_dec2<128>(s, k, grid, adj, in.kv16);
    else launch_dec2<256>(s, k, grid, adj, in.kv16);
  } else if (in.hd == 64) launch_dec<1>(s, k, grid, in.kv16);
  else if (in.hd == 128) launch_dec<2>(s, k, grid, in.kv16);
  else launch_dec<4>(s, k, grid, in.kv16);
  WGD_HIP(hipGetLastError());
  const uint32_t threads = (in.hd + 63) / 64 * 64;
  const uint32_t group = in.kv_heads % 8 == 0 ? k.group : 0;
  hipLaunchKernelGGL(k_attn_comb, dim3(in.heads), dim3(threads), 0, s, (const float *)in.partial, in.y, in.qx,
                     in.pos, in.window, k.chunk, k.nsplit, in.hd, group);
  return hipGetLastError();
}

}  // namespace wgd
