// sample.hip — temperature / top-k / top-p sampling of one logits row on the device.
//
// Replaces sample() (src/core/engine.ts:305-324), whose steps it keeps:
//   * the best finite logit (first index of the maximum; none finite is an error);
//   * temperature 0: that index;
//   * the top-k finite logits in descending order, ties to the lower index (the order the
//     reference's stable insertion sort leaves);
//   * probabilities exp((l - best) / T) in f64, their sum, the shortest prefix whose share
//     reaches top-p, and a draw u * retained walked down that prefix.
// Math.random() becomes the index-th output of splitmix64(seed) (Steele, Lea and Flood,
// "Fast splittable pseudorandom number generators", OOPSLA 2014), scaled to [0, 1) with 53
// bits: the index is the position the sampled token will take, so a sequence is the same
// whether it is decoded one token per call, in device chunks or by graph replays.
//
// One workgroup of 1024 threads. Every finite logit gets a unique 64-bit composite: an
// order-preserving 32-bit key of its value above the complement of its index, so larger
// composites are larger logits and, among equal logits, lower indices. Pass A counts the
// finite logits, finds the largest composite and histograms the top 12 composite bits
// (4096 bins, LDS atomics); a block scan finds the bin holding the k-th largest. If the
// bins above it and it hold at most 1024 composites, pass B gathers them into LDS;
// otherwise the next 12 bits of that bin are histogrammed the same way (values that tie
// over many indices), until they fit. Each gathered composite's rank among them orders them.
#include "internal.h"
#include "decode.h"

namespace wgd {

constexpr uint32_t SMP_T = 1024, SMP_BINS = 4096, SMP_CAND = 1024;

__host__ __device__ inline uint64_t splitmix64_at(uint64_t seed, uint64_t index) {
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Order-preserving key of a finite float (-0 and +0 equal, as the reference compares them).
__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7FFFFFFFu) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ bool finite_f(float v) { return (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u; }
__device__ __forceinline__ uint64_t composite(float v, uint32_t i) {
  return ((uint64_t)order_key(v) << 32) | (0xFFFFFFFFu - i);
}
__device__ __forceinline__ uint32_t comp_index(uint64_t c) { return 0xFFFFFFFFu - (uint32_t)c; }

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return v;
}

// SMP_E logits per thread per step: SMP_E / 4 16-byte loads issued before any is used (one
// workgroup's passes are bound by the round trip of each step: 256 KB per step keeps a
// 128K-entry row to two), element e of the step at index base + 4 * (j * SMP_T + tid) + c
// for e = 4 j + c. Entries past n read as NaN (not finite).
constexpr int SMP_E = 64;
constexpr uint32_t SMP_STEP = SMP_E * SMP_T;
__device__ __forceinline__ void load_step(const float *logits, uint32_t n, uint32_t base, uint32_t tid,
                                          float (&v)[SMP_E]) {
#pragma unroll
  for (int j = 0; j < SMP_E / 4; j++) {
    const uint32_t i = base + 4 * (j * SMP_T + tid);
    if (i + 3 < n) {
      const float4 q = *(const float4 *)(logits + i);
      v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) v[4 * j + c] = i + c < n ? logits[i + c] : __uint_as_float(0x7FC00000u);
    }
  }
}
__device__ __forceinline__ uint32_t at_step(uint32_t base, uint32_t tid, int e) {
  return base + 4 * ((e >> 2) * SMP_T + tid) + (e & 3);
}

struct SampleLds {
  uint32_t hist[SMP_BINS];
  uint64_t cand[SMP_CAND];
  double prob[256];
  uint32_t wsum[16];
  uint64_t wmax[16];
  uint32_t bin, above, ncand, done;
};

// The token for one logits row; st (optional) receives it as k_argmax_advance would.
__global__ __launch_bounds__(SMP_T) void k_sample(const float *logits, uint32_t n, const SampleParams *prm, int32_t index,
                                                  StepState *st, int32_t *out, int32_t *tokens, uint32_t cap,
                                                  int advance) {
  __shared__ SampleLds L;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const SampleParams p = *prm;
  // pass A: finite count, best composite, histogram of bits 63..52
  for (uint32_t b = tid; b < SMP_BINS; b += SMP_T) L.hist[b] = 0;
  __syncthreads();
  // 32-bit keys here (the passes are VALU-bound in one workgroup): a thread visits its
  // indices in increasing order, so a strict > keeps its first maximum
  uint32_t cnt = 0, bkey = 0, bidx = 0;
  for (uint32_t base = 0; base < n; base += SMP_STEP) {
    float v[SMP_E];
    load_step(logits, n, base, tid, v);
#pragma unroll
    for (int e = 0; e < SMP_E; e++) {
      if (!finite_f(v[e])) continue;
      const uint32_t k = order_key(v[e]);
      if (k > bkey) { bkey = k; bidx = at_step(base, tid, e); }
      cnt++;
      atomicAdd(&L.hist[k >> 20], 1u);
    }
  }
  uint64_t best = bkey ? ((uint64_t)bkey << 32) | (0xFFFFFFFFu - bidx) : 0;
  cnt = wave_sum_u32(cnt);
  best = wave_max_u64(best);
  if (lane == 0) { L.wsum[wv] = cnt; L.wmax[wv] = best; }
  __syncthreads();
  cnt = 0; best = 0;
  for (uint32_t w = 0; w < SMP_T / 64; w++) {
    cnt += L.wsum[w];
    best = L.wmax[w] > best ? L.wmax[w] : best;
  }
  int32_t token = -1;
  const bool greedy = p.temperature == 0.0;
  if (cnt > 0 && !greedy) {
    const uint32_t K = p.top_k < cnt ? p.top_k : cnt;
    // Refine until the bin holding the K-th largest, and everything above it, fits in LDS.
    uint64_t prefix = 0;   // composite bits fixed so far
    uint32_t shift = 52;   // the current field starts here: 12 bits, the last one 4 (bits 3..0)
    uint32_t above = 0;    // composites above the current prefix range: all in the top K
    for (;;) {
      // each thread owns four consecutive bins; counts above them from suffix sums over the
      // lanes (shuffles down) and the wavefronts (LDS)
      const uint32_t b0 = 4 * tid;
      const uint32_t s4 = L.hist[b0] + L.hist[b0 + 1] + L.hist[b0 + 2] + L.hist[b0 + 3];
      uint32_t incl = s4;  // becomes the sum of s4 over this and the higher lanes
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t w = __shfl_down(incl, o);
        if (lane + o < 64) incl += w;
      }
      __syncthreads();
      if (lane == 0) L.wsum[wv] = incl;  // the wavefront's total
      __syncthreads();
      uint32_t higher = above + incl - s4;  // composites in the bins above this thread's four
      for (uint32_t w = wv + 1; w < SMP_T / 64; w++) higher += L.wsum[w];
      if (higher < K && higher + s4 >= K) {
        uint32_t h = higher;
        for (int j = 3; j >= 0; j--) {
          const uint32_t c = L.hist[b0 + j];
          if (h + c >= K) { L.bin = b0 + j; L.above = h; break; }
          h += c;
        }
      }
      __syncthreads();
      const uint32_t bin = L.bin;
      above = L.above;
      const uint32_t inbin = L.hist[bin];
      prefix |= (uint64_t)bin << shift;
      __syncthreads();
      if (above + inbin <= SMP_CAND || shift == 0) break;
      // histogram the next field of the bin's composites
      const uint32_t nshift = shift >= 12 ? shift - 12 : 0;
      const uint64_t hi_mask = ~((1ull << shift) - 1);  // bits fixed so far
      const uint32_t fmask = shift >= 12 ? 0xFFFu : (1u << shift) - 1;  // the next field's width
      for (uint32_t b = tid; b < SMP_BINS; b += SMP_T) L.hist[b] = 0;
      __syncthreads();
      for (uint32_t base = 0; base < n; base += SMP_STEP) {
        float v[SMP_E];
        load_step(logits, n, base, tid, v);
#pragma unroll
        for (int e = 0; e < SMP_E; e++) {
          if (!finite_f(v[e])) continue;
          const uint64_t c = composite(v[e], at_step(base, tid, e));
          if ((c & hi_mask) == prefix) atomicAdd(&L.hist[(uint32_t)((c >> nshift) & fmask)], 1u);
        }
      }
      __syncthreads();
      shift = nshift;
    }
    // pass B: every composite at or above the selected bin's range start
    const uint64_t lo = prefix;  // prefix has zeros below the current field
    if (tid == 0) L.ncand = 0;
    for (uint32_t j = tid; j < SMP_CAND; j += SMP_T) L.cand[j] = 0;
    __syncthreads();
    // without refinement the bound has no index bits: compare the 32-bit keys
    const bool keys_only = (lo & 0xFFFFFFFFull) == 0;
    const uint32_t lo_key = (uint32_t)(lo >> 32);
    for (uint32_t base = 0; base < n; base += SMP_STEP) {
      float v[SMP_E];
      load_step(logits, n, base, tid, v);
#pragma unroll
      for (int e = 0; e < SMP_E; e++) {
        const bool fin = finite_f(v[e]);
        const uint32_t k = fin ? order_key(v[e]) : 0;
        const bool pre = fin && k >= lo_key;  // a superset of the composites >= lo
        const uint64_t c = pre ? ((uint64_t)k << 32) | (0xFFFFFFFFu - at_step(base, tid, e)) : 0;
        const bool take = pre && (keys_only || c >= lo);
        const uint64_t m = __ballot(take);
        if (m) {
          uint32_t slot0 = 0;
          if (lane == 0) slot0 = atomicAdd(&L.ncand, (uint32_t)__popcll(m));
          slot0 = __shfl(slot0, 0);
          const uint32_t slot = slot0 + (uint32_t)__popcll(m & ((1ull << lane) - 1));
          if (take && slot < SMP_CAND) L.cand[slot] = c;
        }
      }
    }
    __syncthreads();
    // rank sort, descending: the composites are unique, so each one's place is the count of
    // larger ones (one barrier instead of a sorting network's)
    const uint32_t nc = L.ncand < SMP_CAND ? L.ncand : SMP_CAND;
    uint64_t mine = 0;
    uint32_t rank = 0;
    if (tid < nc) {
      mine = L.cand[tid];
      for (uint32_t j = 0; j < nc; j++) rank += L.cand[j] > mine ? 1u : 0u;
    }
    __syncthreads();
    if (tid < nc) L.cand[rank] = mine;
    __syncthreads();
    // probabilities of the top K (f64, as the reference's numbers)
    const double bestv = (double)logits[comp_index(best)];
    if (tid < K) L.prob[tid] = exp(((double)logits[comp_index(L.cand[tid])] - bestv) / p.temperature);
    __syncthreads();
    if (tid == 0) {
      double total = 0.0;
      for (uint32_t j = 0; j < K; j++) total += L.prob[j];
      double retained = 0.0;
      uint32_t cutoff = 0;
      for (; cutoff < K; cutoff++) {
        retained += L.prob[cutoff];
        if (retained / total >= p.top_p) { cutoff++; break; }
      }
      const int64_t at = index >= 0 ? (int64_t)index : (int64_t)st->pos + 1;
      const double u = (double)(splitmix64_at(p.seed, (uint64_t)at) >> 11) * 0x1.0p-53;
      double draw = u * retained;
      token = (int32_t)comp_index(best);
      for (uint32_t j = 0; j < cutoff; j++) {
        draw -= L.prob[j];
        if (draw <= 0.0) { token = (int32_t)comp_index(L.cand[j]); break; }
      }
    }
  } else if (cnt > 0) {
    token = (int32_t)comp_index(best);
  }
  if (tid != 0) return;
  *out = token;
  if (!advance) return;
  int32_t t = token;
  if (t < 0) { st->error = 1; t = 0; }
  if ((uint32_t)st->step < cap) tokens[st->step] = t;
  st->token = t;
  st->pos += 1;
  st->step += 1;
}

hipError_t sample(hipStream_t s, const float *logits, uint32_t n, const SampleParams *params, int32_t index,
                  StepState *st, int32_t *out, int32_t *tokens, uint32_t cap, bool advance) {
  if (!n || (index < 0 && !st) || (advance && (!st || !tokens))) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(SMP_T), 0, s, logits, n, params, index, st, out, tokens, cap,
                     advance ? 1 : 0);
  return hipGetLastError();
}

}  // namespace wgd
