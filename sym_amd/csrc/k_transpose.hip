// k_transpose.hip - LDS-tiled transpose kernels.
#include "kernels.h"

namespace relx {
namespace {

} // namespace
RELX_DISPATCH_FAST(transpose_fast, transpose_launch)
RELX_DISPATCH_GENERIC(transpose_generic, transpose_launch)

} // namespace relx
