// kernels.hip - the generic kernel's launch and the family dispatcher.
// Kernel bodies live in kernels.h; the fast families are instantiated in
// k_stream_fast.hip, k_stream_generic.hip, k_transpose.hip, k_interleave.hip,
// k_interleave_generic.hip, k_permute.hip.
#include "kernels.h"

namespace relx {

// Launch one box of a program. `status` is a device int the generic kernel
// sets when a channel index falls outside its parameter table.
hipError_t launch_box(int family, const KArgs &a, int32_t *status, hipStream_t s) {
  if (a.work64 <= 0)
    return hipSuccess;
  bool handled = false;
  hipError_t e = hipSuccess;
  switch (family) {
  case kFamStream:
    e = stream_fast(a, s, handled);
    return handled ? e : stream_generic(a, s);
  case kFamTranspose:
    e = transpose_fast(a, s, handled);
    return handled ? e : transpose_generic(a, s);
  case kFamInterleave:
    e = interleave_fast(a, s, handled);
    return handled ? e : interleave_generic(a, s);
  case kFamPermute:
    e = permute_fast(a, s, handled);
    return handled ? e : permute_generic(a, s);
  default:
    hipLaunchKernelGGL(k_generic, dim3(grid_for(a.work64)), dim3(kBlock), 0, s, a, status);
    return hipGetLastError();
  }
}

} // namespace relx
