// probe.hip — a plain streaming read of a device buffer, the per-launch floor that any kernel
// reading `bytes` once meets on this hardware: 16-byte non-temporal buffer loads, `depth` of
// them in flight per lane, a contiguous range per workgroup, no arithmetic beyond an xor that
// keeps the loads live. With out_floats > 0 each workgroup also stores its share of an
// out_floats-long result vector, as a matvec stores one float per output row. Measurement
// only: the matvec microbench reports its launches against this floor.
#include "internal.h"

namespace wgd {

typedef unsigned int probe_u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(1024) void k_probe_read(const uint8_t *p, uint32_t bytes, uint32_t chunk, float *out,
                                                     uint32_t out_n) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)bytes, 0x00020000);
  const uint32_t nt = blockDim.x, tid = threadIdx.x;
  const uint32_t lo = blockIdx.x * chunk, hi = lo + chunk;  // 16-byte pieces of this workgroup
  uint32_t acc = 0;
  for (uint32_t i = lo + tid; i < hi; i += nt * U) {
    probe_u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t e = i + u * nt;
      // pieces past the range read offset `bytes`, which the buffer bound turns into zeros
      v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, e < hi ? e * 16 : bytes, 0, 2);
    }
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (out_n) {
    // this workgroup's share of the result: out[o] for o in [o0, o1)
    const uint32_t per = (out_n + gridDim.x - 1) / gridDim.x, o0 = blockIdx.x * per;
    const uint32_t o1 = o0 + per < out_n ? o0 + per : out_n;
    for (uint32_t o = o0 + tid; o < o1; o += nt) out[o] = __uint_as_float(acc & 0x3f7fffffu);
  } else if (acc == 0x9e3779b9u && out) {
    out[0] = 0.f;  // never taken in practice; keeps the loads from being removed
  }
}

hipError_t probe_read(hipStream_t s, const uint8_t *p, uint32_t bytes, uint32_t wgs, uint32_t threads, uint32_t depth,
                      float *out, uint32_t out_n) {
  if (!wgs || !threads || threads % 64 || threads > 1024 || bytes % 16 || !bytes) return hipErrorInvalidValue;
  const uint32_t chunk = (bytes / 16 + wgs - 1) / wgs;
  switch (depth) {
    case 4: hipLaunchKernelGGL(k_probe_read<4>, dim3(wgs), dim3(threads), 0, s, p, bytes, chunk, out, out_n); break;
    case 8: hipLaunchKernelGGL(k_probe_read<8>, dim3(wgs), dim3(threads), 0, s, p, bytes, chunk, out, out_n); break;
    case 16: hipLaunchKernelGGL(k_probe_read<16>, dim3(wgs), dim3(threads), 0, s, p, bytes, chunk, out, out_n); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace wgd
