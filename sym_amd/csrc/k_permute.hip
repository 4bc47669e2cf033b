// k_permute.hip - LDS block-permute kernels.
#include "kernels.h"

namespace relx {
namespace {

} // namespace
RELX_DISPATCH_FAST(permute_fast, permute_launch)
RELX_DISPATCH_GENERIC(permute_generic, permute_launch)

} // namespace relx
