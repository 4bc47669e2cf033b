// k_copy.hip - a plain 16-byte vector copy, used only to measure the HBM
// copy ceiling the relayout kernels are compared against (same access shape
// as the stream kernel: two 16-byte items per lane, 64 apart, streamed past
// the caches).
#include "kernels.h"

namespace relx {
namespace {

__global__ __launch_bounds__(kBlock) void k_copy16(const vec4 *src, vec4 *dst, uint32_t n) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = (blockIdx.x * kBlock + threadIdx.x) >> 6;
  const uint32_t stride = gridDim.x * (kBlock / 64) * 128u;
  for (uint32_t base = wave * 128u + lane; base < n; base += stride) {
    const uint32_t i1 = base + 64u;
    const bool live = i1 < n;
    const vec4 a = ld16<true>(src + base);
    vec4 b = {0u, 0u, 0u, 0u};
    if (live)
      b = ld16<true>(src + i1);
    st16<true>(dst + base, a);
    if (live)
      st16<true>(dst + i1, b);
  }
}

} // namespace

// Copy `n16` 16-byte vectors (n16 < 2^31) from src to dst on `s`.
hipError_t copy16_launch(const void *src, void *dst, uint32_t n16, hipStream_t s) {
  if (n16 == 0)
    return hipSuccess;
  hipLaunchKernelGGL(k_copy16, dim3(grid_for((static_cast<int64_t>(n16) + 1) / 2)), dim3(kBlock), 0,
                     s, static_cast<const vec4 *>(src), static_cast<vec4 *>(dst), n16);
  return hipGetLastError();
}

} // namespace relx
