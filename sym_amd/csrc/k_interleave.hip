// k_interleave.hip - planar -> interleaved kernels, per-tensor chains.
#include "kernels.h"

namespace relx {
RELX_DISPATCH_FAST(interleave_fast, interleave_launch)
} // namespace relx
