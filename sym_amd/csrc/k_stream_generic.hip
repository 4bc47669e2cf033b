// k_stream_generic.hip - stream kernels with per-stage dispatch.
#include "kernels.h"

namespace relx {
namespace {

} // namespace
RELX_DISPATCH_GENERIC(stream_generic, stream_launch)

} // namespace relx
