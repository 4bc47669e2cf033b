// noalloc.hip - the device scratch of the allocation-free upload
// (relx_execute_h2d_static).
//
// Callers that cannot allocate device memory (tight serving loops,
// harnesses that forbid allocation) get an upload whose staging lives in
// this file-scope array instead of the context's wire arena: each GPU the
// library runs on holds its own copy of it, of kScratchBytes, until the
// process ends. Host code never passes `scratch` itself to a kernel or a
// copy (on the host the name is only a stand-in for the symbol): it takes
// the device address of the current GPU's copy from hipGetSymbolAddress,
// once per device, and uses that.
#include "runtime.h"

#include <map>
#include <memory>
#include <mutex>

namespace relx {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_static_mu;
std::map<int, std::unique_ptr<StaticDevice>> g_static; // device -> its state
} // namespace

StaticDevice &static_device(int device) {
  std::lock_guard<std::mutex> g(g_static_mu);
  auto it = g_static.find(device);
  if (it != g_static.end())
    return *it->second;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != device)
    throw Error("backend_failure", "the static scratch is looked up with its device current");
  void *p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    throw Error("backend_failure",
                std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  auto st = std::make_unique<StaticDevice>();
  st->addr = static_cast<uint8_t *>(p);
  e = hipEventCreateWithFlags(&st->last, hipEventDisableTiming);
  if (e != hipSuccess)
    throw Error("backend_failure", std::string("hipEventCreateWithFlags: ") + hipGetErrorString(e));
  return *g_static.emplace(device, std::move(st)).first->second;
}

} // namespace relx
