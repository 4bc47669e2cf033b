// noalloc.hip - the device scratch of the allocation-free upload
// (relx_execute_h2d_static).
//
// Callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid allocation) get an upload whose
// staging lives in this file-scope array instead of the context's wire arena:
// each GPU the library runs on holds its own copy of it, of kScratchBytes,
// until the process ends. Host code never passes `scratch` itself to a kernel
// or a copy (on the host the name is only a stand-in for the symbol): it
// takes the device address of the current GPU's copy from
// hipGetSymbolAddress, once per device, and uses that.
#include "runtime.h"

#include <map>
#include <mutex>

namespace relx {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::map<int, uint8_t *> g_scratch_addr; // device -> its copy of `scratch`
} // namespace

uint8_t *scratch_address(int device) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  auto it = g_scratch_addr.find(device);
  if (it != g_scratch_addr.end())
    return it->second;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != device)
    throw Error("backend_failure", "the static scratch is looked up with its device current");
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    throw Error("backend_failure",
                std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  g_scratch_addr.emplace(device, static_cast<uint8_t *>(p));
  return static_cast<uint8_t *>(p);
}

} // namespace relx
