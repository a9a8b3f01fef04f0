// Float32 atomic-add throughput, for the counter-enabled measurement build only (THERIA_TILE_COUNT).
//
// A backward kernel that forms dQ inside the dK/dV kernel would add each workgroup's partial dQ to a float32
// workspace with global atomics, once per key block: at config 2 (B4 H16 S2048 D64) with 256-key blocks that is
// 8 x 33.5 MB. This kernel issues the same pattern (one 256-thread workgroup adds to 128 rows x 64 columns of a
// dQ-sized buffer, `reps` workgroups per rows block, consecutive workgroups on different blocks, coalesced
// 256-byte wave accesses) as relaxed device-scope atomics, or as plain stores of the same shape, so that the
// time of the atomics alone can be set against the dQ kernel they would replace.
#ifdef THERIA_TILE_COUNT
#include "sdpa_common.hpp"

namespace theria {

constexpr int kProbeChunk = 128 * 64;  // floats per workgroup

template <bool ATOMIC>
__global__ __launch_bounds__(256) void atomic_probe_kernel(float* __restrict__ buf, int nchunk) {
  const int chunk = blockIdx.x % nchunk;  // < nchunk: every access lies in [0, nchunk * kProbeChunk)
  float* base = buf + (int64_t)chunk * kProbeChunk;
  const float v = 1.0f + 0.001f * (float)(blockIdx.x / nchunk);
#pragma unroll
  for (int i = 0; i < kProbeChunk / 256; ++i) {
    float* p = base + i * 256 + threadIdx.x;
    if constexpr (ATOMIC)
      __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      *p = v;
  }
}

hipError_t launch_atomic_probe(float* buf, int64_t n, int reps, bool atomic, hipStream_t st) {
  const int64_t nchunk = n / kProbeChunk;
  if (nchunk <= 0 || reps <= 0 || nchunk * reps > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(nchunk * reps)), block(256);
  if (atomic)
    hipLaunchKernelGGL((atomic_probe_kernel<true>), grid, block, 0, st, buf, (int)nchunk);
  else
    hipLaunchKernelGGL((atomic_probe_kernel<false>), grid, block, 0, st, buf, (int)nchunk);
  return hipGetLastError();
}

}  // namespace theria
#endif
