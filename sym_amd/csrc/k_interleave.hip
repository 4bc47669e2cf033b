// k_interleave.hip - planar -> interleaved kernels.
#include "kernels.h"

namespace relx {
namespace {

} // namespace
RELX_DISPATCH_FAST(interleave_fast, interleave_launch)
RELX_DISPATCH_GENERIC(interleave_generic, interleave_launch)

} // namespace relx
