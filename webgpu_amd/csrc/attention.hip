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

namespace wgd {

struct AttnK {
  const float *q, *k, *v; float *y, *part;
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
        kvk = a.k[src]; kvv = a.v[src];
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

__global__ __launch_bounds__(128) void k_attention_combine(const float *part, float *y, uint32_t rows,
                                                           uint32_t hd, uint32_t nsplit) {
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
    y[row * hd + d] = L > 0.f ? acc / L : 0.f;
  }
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

hipError_t attention(hipStream_t s, const AttnArgs &in) {
  if (!in.batch) return hipSuccess;
  if (!in.kv_heads || in.heads % in.kv_heads || in.hd == 0 || in.hd > 512 || !in.capacity || !in.window)
    return hipErrorInvalidValue;
  AttnK a;
  a.q = in.q; a.k = in.k; a.v = in.v; a.y = in.y; a.part = in.partial;
  a.heads = in.heads; a.kvh = in.kv_heads; a.hd = in.hd; a.start = in.start; a.start_dev = in.start_dev;
  a.scale = in.scale; a.window = in.window; a.capacity = in.capacity; a.batch = in.batch;
  a.group = in.heads / in.kv_heads;
  a.qb = a.group >= 16 ? 1 : 16 / a.group;
  if (a.qb > in.batch) a.qb = in.batch;
  a.R = a.qb * a.group;
  if (a.R > 16) return hipErrorInvalidValue;
  a.T = tile_keys(in.hd);
  const uint32_t qblocks = (in.batch + a.qb - 1) / a.qb;
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
  uint32_t tiles = (keys + a.T - 1) / a.T;
  uint32_t want = (uint32_t)device_cu_count() * 4 / (in.kv_heads * qblocks);
  uint32_t nsplit = tiles < want ? tiles : want;
  if (nsplit < 1) nsplit = 1;
  if (nsplit > 1) {
    uint64_t per_split = (uint64_t)in.batch * in.heads * (in.hd + 2);
    uint64_t fit = in.partial ? in.partial_floats / per_split : 0;
    if (fit < nsplit) nsplit = fit > 1 ? (uint32_t)fit : 1;
  }
  a.nsplit = nsplit;
  size_t lds = sizeof(float) * ((size_t)a.T * (in.hd + 1) + (size_t)a.T * in.hd + (size_t)a.R * in.hd +
                                (size_t)a.R * a.T + 3 * a.R);
  static bool big_lds = false;
  if (lds > 65536 && !big_lds) {
    (void)hipFuncSetAttribute((const void *)k_attention, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    big_lds = true;
  }
  hipLaunchKernelGGL(k_attention, dim3(in.kv_heads, qblocks, nsplit), dim3(256), lds, s, a);
  WGD_HIP(hipGetLastError());
  if (nsplit > 1) {
    hipLaunchKernelGGL(k_attention_combine, dim3(in.batch * in.heads), dim3(128), 0, s, (const float *)in.partial,
                       in.y, in.batch * in.heads, in.hd, nsplit);
    WGD_HIP(hipGetLastError());
  }
  return hipSuccess;
}

}  // namespace wgd
