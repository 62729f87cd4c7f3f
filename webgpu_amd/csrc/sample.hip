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
// Every finite logit has a unique 64-bit composite: an order-preserving 32-bit key of its
// value above the complement of its index, so larger composites are larger logits and,
// among equal logits, lower indices. Two launches:
//   * k_sample_local, one workgroup per slice of about 2K logits (one workgroup's loads
//     cannot stream a 500 KB row quickly): the slice's finite count and best composite, a
//     histogram of the top 12 key bits, and every composite at or above the bin holding the
//     slice's k-th largest. That is a superset of the slice's top k, so together the slices
//     hold the row's top k.
//   * k_sample, one workgroup of 1024 threads over those candidates: a 4096-bin histogram of
//     the top 12 composite bits and a block scan find the bin holding the k-th largest; if it
//     and the bins above hold at most 1024 candidates they are gathered into LDS, otherwise
//     the next 12 bits of that bin are histogrammed (values that tie over many indices) until
//     they fit. Each gathered composite's rank orders them; then the probabilities and draw.
#include "internal.h"
#include "decode.h"

namespace wgd {

constexpr uint32_t SMP_T = 1024, SMP_BINS = 4096, SMP_CAND = 1024;
constexpr uint32_t SL_T = 256, SL_MAX = 256, SL_SLICE = 1024;  // local kernel: threads, slices, slice floor
constexpr uint32_t SL_E = 4;  // logits per thread per step of the local kernel, loaded before use
constexpr uint32_t SMP_R = 16;  // candidates per thread held in registers by the selection

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

// The bin of hist[0..NB) holding the K-th largest entry when `above` entries are larger
// than every bin, and the count above that bin, to *out_bin / *out_above. Each of the T
// threads owns NB / T consecutive bins. Every thread calls it; K <= above + the total.
template <uint32_t T, uint32_t NB>
__device__ __forceinline__ void find_bin(const uint32_t *hist, uint32_t above, uint32_t K, uint32_t *wsum,
                                         uint32_t *out_bin, uint32_t *out_above) {
  constexpr uint32_t PER = NB / T;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t b0 = PER * tid;
  uint32_t s = 0;
#pragma unroll
  for (uint32_t j = 0; j < PER; j++) s += hist[b0 + j];
  uint32_t incl = s;  // the sum of s over this and the higher lanes
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t w = __shfl_down(incl, o);
    if (lane + o < 64) incl += w;
  }
  __syncthreads();
  if (lane == 0) wsum[wv] = incl;
  __syncthreads();
  uint32_t higher = above + incl - s;  // entries in the bins above this thread's
  for (uint32_t w = wv + 1; w < T / 64; w++) higher += wsum[w];
  if (higher < K && higher + s >= K) {
    uint32_t h = higher;
    for (int j = (int)PER - 1; j >= 0; j--) {
      const uint32_t c = hist[b0 + j];
      if (h + c >= K) { *out_bin = b0 + j; *out_above = h; break; }
      h += c;
    }
  }
  __syncthreads();
}

// ------------------------------------------------------------------ per-slice candidates

struct SliceOut { uint64_t best; uint32_t finite, count; };

__global__ __launch_bounds__(SL_T) void k_sample_local(const float *logits, uint32_t n, uint32_t slice,
                                                       const SampleParams *prm, uint64_t *cand, SliceOut *so) {
  __shared__ uint32_t hist[SMP_BINS];
  __shared__ uint32_t wsum[SL_T / 64];
  __shared__ uint64_t wmax[SL_T / 64];
  __shared__ uint32_t sh_bin, sh_above, sh_count;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, w = blockIdx.x;
  const uint32_t lo = w * slice, hi = lo + slice < n ? lo + slice : n;
  for (uint32_t b = tid; b < SMP_BINS; b += SL_T) hist[b] = 0;
  if (tid == 0) { sh_count = 0; sh_bin = 0; sh_above = 0; }
  __syncthreads();
  // the slice is read twice; the second time from this CU's caches
  uint32_t cnt = 0;
  uint64_t best = 0;
  for (uint32_t i0 = lo; i0 < hi; i0 += SL_T * SL_E) {
    float v[SL_E];
#pragma unroll
    for (uint32_t e = 0; e < SL_E; e++) {
      const uint32_t i = i0 + e * SL_T + tid;
      v[e] = i < hi ? logits[i] : __uint_as_float(0x7FC00000u);
    }
#pragma unroll
    for (uint32_t e = 0; e < SL_E; e++) {
      if (!finite_f(v[e])) continue;
      const uint32_t i = i0 + e * SL_T + tid;
      const uint32_t k = order_key(v[e]);
      const uint64_t c = ((uint64_t)k << 32) | (0xFFFFFFFFu - i);
      best = c > best ? c : best;
      cnt++;
      atomicAdd(&hist[k >> 20], 1u);
    }
  }
  cnt = wave_sum_u32(cnt);
  best = wave_max_u64(best);
  if (lane == 0) { wsum[wv] = cnt; wmax[wv] = best; }
  __syncthreads();
  cnt = 0; best = 0;
  for (uint32_t u = 0; u < SL_T / 64; u++) {
    cnt += wsum[u];
    best = wmax[u] > best ? wmax[u] : best;
  }
  const SampleParams p = *prm;
  const uint32_t K = p.top_k < cnt ? p.top_k : cnt;
  const bool gather = p.temperature != 0.0 && K > 0;
  if (gather) {
    find_bin<SL_T, SMP_BINS>(hist, 0, K, wsum, &sh_bin, &sh_above);
    const uint32_t lo_key = sh_bin << 20;
    uint64_t *out = cand + (uint64_t)w * slice;
    for (uint32_t i0 = lo; i0 < hi; i0 += SL_T) {
      const uint32_t i = i0 + tid;
      const float v = i < hi ? logits[i] : __uint_as_float(0x7FC00000u);
      const bool fin = finite_f(v);
      const uint32_t k = fin ? order_key(v) : 0;
      const bool take = fin && k >= lo_key;
      const uint64_t m = __ballot(take);
      if (m) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&sh_count, (uint32_t)__popcll(m));
        base = __shfl(base, 0);
        if (take) out[base + (uint32_t)__popcll(m & ((1ull << lane) - 1))] = ((uint64_t)k << 32) | (0xFFFFFFFFu - i);
      }
    }
    __syncthreads();
  }
  if (tid == 0) so[w] = SliceOut{best, cnt, gather ? sh_count : 0u};
}

// ------------------------------------------------------------------ selection and draw

struct SampleLds {
  uint32_t hist[SMP_BINS];
  uint64_t cand[SMP_CAND];
  double prob[256];
  uint32_t offs[SL_MAX + 1];
  uint32_t wsum[16];
  uint64_t wmax[16];
  uint32_t bin, above, ncand;
};

// The token from the slices' candidates; st (optional) receives it as k_argmax_advance would.
__global__ __launch_bounds__(SMP_T) void k_sample(const float *logits, const uint64_t *cand, const SliceOut *so,
                                                  uint32_t nslices, uint32_t slice, const SampleParams *prm,
                                                  int32_t index, StepState *st, int32_t *out, int32_t *tokens,
                                                  uint32_t cap, int advance) {
  __shared__ SampleLds L;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const SampleParams p = *prm;
  // the slices' totals, and the offsets of their candidate lists in one flat range [0, C):
  // one summary per thread (all loads at once), then a scan by thread 0 in LDS
  const SliceOut mine_so = tid < nslices ? so[tid] : SliceOut{0, 0, 0};
  if (tid < nslices) L.offs[tid + 1] = mine_so.count;
  uint32_t cnt = wave_sum_u32(mine_so.finite);
  uint64_t best = wave_max_u64(mine_so.best);
  if (lane == 0) { L.wsum[tid >> 6] = cnt; L.wmax[tid >> 6] = best; }
  __syncthreads();
  if (tid == 0) {
    L.offs[0] = 0;
    for (uint32_t w = 0; w < nslices; w++) L.offs[w + 1] += L.offs[w];
  }
  cnt = 0; best = 0;
  for (uint32_t u = 0; u < SMP_T / 64; u++) {
    cnt += L.wsum[u];
    best = L.wmax[u] > best ? L.wmax[u] : best;
  }
  __syncthreads();
  const uint32_t C = L.offs[nslices];
  auto at = [&](uint32_t i) -> uint64_t {  // flat candidate i: binary search over the offsets
    uint32_t a = 0, b = nslices;
    while (b - a > 1) {
      const uint32_t mid = (a + b) >> 1;
      if (L.offs[mid] <= i) a = mid; else b = mid;
    }
    return cand[(uint64_t)a * slice + (i - L.offs[a])];
  };
  // The candidates, loaded once: all loads issued together, then kept in registers for every
  // pass (up to SMP_T * SMP_R of them; more are read again per pass).
  const bool resident = C <= SMP_T * SMP_R;
  uint64_t cr[SMP_R];
#pragma unroll
  for (uint32_t r = 0; r < SMP_R; r++) {
    const uint32_t i = r * SMP_T + tid;
    cr[r] = resident && i < C ? at(i) : 0;
  }
  // f(c) over every candidate c this thread owns (uniform control flow: f may use ballots)
  auto each = [&](auto f) {
    if (resident) {
#pragma unroll
      for (uint32_t r = 0; r < SMP_R; r++) {
        const uint32_t i = r * SMP_T + tid;
        f(i < C, cr[r]);
      }
    } else {
      for (uint32_t i0 = 0; i0 < C; i0 += SMP_T) {
        const uint32_t i = i0 + tid;
        f(i < C, i < C ? at(i) : 0);
      }
    }
  };
  int32_t token = -1;
  if (cnt > 0 && p.temperature == 0.0) {
    token = (int32_t)comp_index(best);
  } else if (cnt > 0) {
    const uint32_t K = p.top_k < cnt ? p.top_k : cnt;
    for (uint32_t b = tid; b < SMP_BINS; b += SMP_T) L.hist[b] = 0;
    __syncthreads();
    each([&](bool ok, uint64_t c) { if (ok) atomicAdd(&L.hist[c >> 52], 1u); });
    __syncthreads();
    // refine until the bin holding the K-th largest, and everything above it, fits in LDS
    uint64_t prefix = 0;   // composite bits fixed so far
    uint32_t shift = 52;   // the current field starts here: 12 bits, the last one 4 (bits 3..0)
    uint32_t above = 0;    // candidates above the current prefix range: all in the top K
    for (;;) {
      find_bin<SMP_T, SMP_BINS>(L.hist, above, K, L.wsum, &L.bin, &L.above);
      const uint32_t bin = L.bin;
      above = L.above;
      const uint32_t inbin = L.hist[bin];
      prefix |= (uint64_t)bin << shift;
      __syncthreads();
      if (above + inbin <= SMP_CAND || shift == 0) break;
      const uint32_t nshift = shift >= 12 ? shift - 12 : 0;
      const uint64_t hi_mask = ~((1ull << shift) - 1);                   // bits fixed so far
      const uint32_t fmask = shift >= 12 ? 0xFFFu : (1u << shift) - 1;  // the next field's width
      for (uint32_t b = tid; b < SMP_BINS; b += SMP_T) L.hist[b] = 0;
      __syncthreads();
      each([&](bool ok, uint64_t c) {
        if (ok && (c & hi_mask) == prefix) atomicAdd(&L.hist[(uint32_t)((c >> nshift) & fmask)], 1u);
      });
      __syncthreads();
      shift = nshift;
    }
    // every candidate at or above the selected bin's range start (prefix: zeros below it)
    if (tid == 0) L.ncand = 0;
    __syncthreads();
    each([&](bool ok, uint64_t c) {
      const bool take = ok && c >= prefix;
      const uint64_t m = __ballot(take);
      if (m) {
        uint32_t slot0 = 0;
        if (lane == 0) slot0 = atomicAdd(&L.ncand, (uint32_t)__popcll(m));
        slot0 = __shfl(slot0, 0);
        const uint32_t slot = slot0 + (uint32_t)__popcll(m & ((1ull << lane) - 1));
        if (take && slot < SMP_CAND) L.cand[slot] = c;
      }
    });
    __syncthreads();
    // rank sort, descending: the composites are unique, so each one's place is the count of
    // larger ones
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
      const int64_t at_pos = index >= 0 ? (int64_t)index : (int64_t)st->pos + 1;
      const double u = (double)(splitmix64_at(p.seed, (uint64_t)at_pos) >> 11) * 0x1.0p-53;
      double draw = u * retained;
      token = (int32_t)comp_index(best);
      for (uint32_t j = 0; j < cutoff; j++) {
        draw -= L.prob[j];
        if (draw <= 0.0) { token = (int32_t)comp_index(L.cand[j]); break; }
      }
    }
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

// Slices of at least SL_SLICE logits (a multiple of 4), at most SL_MAX of them.
static void slicing(uint32_t n, uint32_t *nslices, uint32_t *slice) {
  uint32_t s = (n + SL_MAX - 1) / SL_MAX;
  if (s < SL_SLICE) s = SL_SLICE;
  s = (s + 3) & ~3u;
  *slice = s;
  *nslices = (n + s - 1) / s;
}

static uint64_t cand_bytes(uint32_t nslices, uint32_t slice) { return ((uint64_t)nslices * slice * 8 + 255) / 256 * 256; }

uint64_t sample_scratch_bytes(uint32_t n) {
  uint32_t ns, sl;
  slicing(n, &ns, &sl);
  return cand_bytes(ns, sl) + SL_MAX * sizeof(SliceOut);
}

hipError_t sample(hipStream_t s, const float *logits, uint32_t n, const SampleParams *params, int32_t index,
                  StepState *st, int32_t *out, int32_t *tokens, uint32_t cap, bool advance, void *scratch) {
  if (!n || !scratch || (index < 0 && !st) || (advance && (!st || !tokens))) return hipErrorInvalidValue;
  uint32_t ns, sl;
  slicing(n, &ns, &sl);
  uint64_t *cand = (uint64_t *)scratch;
  SliceOut *so = (SliceOut *)((uint8_t *)scratch + cand_bytes(ns, sl));
  hipLaunchKernelGGL(k_sample_local, dim3(ns), dim3(SL_T), 0, s, logits, n, sl, params, cand, so);
  WGD_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(SMP_T), 0, s, logits, (const uint64_t *)cand, (const SliceOut *)so, ns,
                     sl, params, index, st, out, tokens, cap, advance ? 1 : 0);
  return hipGetLastError();
}

}  // namespace wgd
