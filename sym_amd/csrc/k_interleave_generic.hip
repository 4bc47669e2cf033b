// k_interleave_generic.hip - planar -> interleaved kernels, generic chains.
#include "kernels.h"

namespace relx {
RELX_DISPATCH_GENERIC(interleave_generic, interleave_launch)
} // namespace relx
