// k_copy.hip - a plain 16-byte vector copy, used only to measure the HBM
// copy ceiling the relayout kernels are compared against (wave-contiguous
// 16-byte vectors streamed past the caches, U per lane 64 apart: one lane
// per vector is the faster form from about 128 MB up, two below).
#include "kernels.h"

namespace relx {
namespace {

template <int U>
__global__ __launch_bounds__(kBlock) void k_copy16(const vec4 *src, vec4 *dst, uint32_t n) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = (blockIdx.x * kBlock + threadIdx.x) >> 6;
  const uint32_t stride = gridDim.x * (kBlock / 64) * (64u * U);
  for (uint32_t base = wave * (64u * U) + lane; base < n; base += stride) {
    vec4 v[U];
    // every load issues before any store; a second item past the end reads
    // the first one again and is not stored
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i = base + 64u * u;
      v[u] = ld16<true>(src + (i < n ? i : base));
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (u == 0 || base + 64u * u < n)
        st16<true>(dst + base + 64u * u, v[u]);
  }
}

} // namespace

// Copy `n16` 16-byte vectors (n16 < 2^31) from src to dst on `s`, `items`
// (1 or 2) vectors per lane.
hipError_t copy16_launch(const void *src, void *dst, uint32_t n16, int items, hipStream_t s) {
  if (n16 == 0)
    return hipSuccess;
  const vec4 *sv = static_cast<const vec4 *>(src);
  vec4 *dv = static_cast<vec4 *>(dst);
  if (items == 1)
    hipLaunchKernelGGL(k_copy16<1>, dim3(grid_for(n16)), dim3(kBlock), 0, s, sv, dv, n16);
  else
    hipLaunchKernelGGL(k_copy16<2>, dim3(grid_for((static_cast<int64_t>(n16) + 1) / 2)),
                       dim3(kBlock), 0, s, sv, dv, n16);
  return hipGetLastError();
}

} // namespace relx
