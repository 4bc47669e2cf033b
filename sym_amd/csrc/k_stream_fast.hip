// k_stream_fast.hip - stream kernels for the compile-time stage chains.
#include "kernels.h"

namespace relx {
namespace {

} // namespace
RELX_DISPATCH_FAST(stream_fast, stream_launch)

} // namespace relx
