// The reference's own CPU H2D path on a HIP copy backend (TEST INFRASTRUCTURE
// ONLY: the CPU baseline that bench.py times; never the product).
//
// The reference writes its transfer pipelines once against the CopyBackend
// plugin interface (libreloc/include/reloc/Backend.h:34-89) and ships a CUDA
// implementation of it. This file implements that interface with the HIP
// runtime (pinned staging, hipMemcpyAsync on its own streams, events), then
// runs the reference's unmodified `cpu_reference` dispatch row through it:
//   prepareDispatch / executeDispatch      libreloc/src/Dispatch.cpp:1558-1620,1983-2046
//   transformToDevice (the 2-slot ring)    libreloc/src/Dispatch.cpp:452-546
//   executeTransfer (layout plans, ring)   libreloc/src/Transfer.cpp:493-544
// so the CPU transform into pinned slots and the H2D of its result are the
// reference's code; only the copy engine is HIP. Built by oracle/Makefile into
// oracle/_ref/libreloc_ref_hip.so, linked against libreloc_ref.so.
#include "reloc/Backend.h"
#include "reloc/Bind.h"
#include "reloc/Decode.h"
#include "reloc/Dispatch.h"
#include "reloc/GatherPool.h"
#include "reloc/Transfer.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace {

class HipCopyBackend final : public reloc::CopyBackend {
public:
  HipCopyBackend(int device, int queues) : device_(device) {
    if (!ok(hipSetDevice(device), "hipSetDevice"))
      return;
    for (int i = 0; i < queues; ++i) {
      hipStream_t s = nullptr;
      if (!ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate"))
        return;
      streams_.push_back(s);
    }
  }
  ~HipCopyBackend() override {
    (void)quiesce();
    for (auto &kv : events_)
      (void)hipEventDestroy(kv.second);
    for (hipStream_t s : streams_)
      (void)hipStreamDestroy(s);
  }

  void *allocStaging(size_t bytes) override {
    void *p = nullptr;
    if (!ok(hipHostMalloc(&p, bytes, hipHostMallocDefault), "hipHostMalloc"))
      return nullptr;
    return p;
  }
  void freeStaging(void *p) override {
    if (p)
      (void)hipHostFree(p);
  }
  int numQueues() const override { return static_cast<int>(streams_.size()); }
  void copyAsync(int queue, void *dst, const void *src, size_t bytes,
                 reloc::CopyDir dir) override {
    if (queue < 0 || queue >= numQueues()) {
      record("copy on a queue that does not exist");
      return;
    }
    ok(hipMemcpyAsync(dst, src, bytes,
                      dir == reloc::CopyDir::HostToDevice ? hipMemcpyHostToDevice
                                                          : hipMemcpyDeviceToHost,
                      streams_[static_cast<size_t>(queue)]),
       "hipMemcpyAsync");
  }
  reloc::EventHandle recordEvent(int queue) override {
    if (queue < 0 || queue >= numQueues())
      return 0;
    hipEvent_t e = nullptr;
    if (!ok(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate"))
      return 0;
    if (!ok(hipEventRecord(e, streams_[static_cast<size_t>(queue)]), "hipEventRecord")) {
      (void)hipEventDestroy(e);
      return 0;
    }
    std::lock_guard<std::mutex> g(mu_);
    const reloc::EventHandle h = next_++;
    events_[h] = e;
    return h;
  }
  void waitEvent(reloc::EventHandle ev) override {
    hipEvent_t e = take(ev);
    if (!e)
      return;
    ok(hipEventSynchronize(e), "hipEventSynchronize");
    (void)hipEventDestroy(e);
  }
  bool queryEvent(reloc::EventHandle ev) override {
    if (ev == 0)
      return true;
    std::lock_guard<std::mutex> g(mu_);
    auto it = events_.find(ev);
    return it == events_.end() || hipEventQuery(it->second) == hipSuccess;
  }
  reloc::QueueCompletion quiesce() override {
    bool all = true;
    for (hipStream_t s : streams_)
      all = hipStreamSynchronize(s) == hipSuccess && all;
    return all ? reloc::QueueCompletion::Complete : reloc::QueueCompletion::Unknown;
  }
  bool waitStream(const void *external) override {
    hipEvent_t e = nullptr;
    if (!ok(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate"))
      return false;
    bool good = ok(hipEventRecord(e, static_cast<hipStream_t>(const_cast<void *>(external))),
                   "hipEventRecord");
    for (hipStream_t s : streams_)
      good = good && ok(hipStreamWaitEvent(s, e, 0), "hipStreamWaitEvent");
    (void)hipEventDestroy(e);
    return good;
  }
  bool failed() const override { return failed_; }
  const std::string &error() const override { return error_; }
  int device() const override { return device_; }

private:
  bool ok(hipError_t e, const char *what) {
    if (e == hipSuccess)
      return true;
    record(std::string(what) + ": " + hipGetErrorString(e));
    return false;
  }
  void record(const std::string &msg) {
    if (!failed_) {
      failed_ = true;
      error_ = msg;
    }
  }
  hipEvent_t take(reloc::EventHandle ev) {
    if (ev == 0)
      return nullptr;
    std::lock_guard<std::mutex> g(mu_);
    auto it = events_.find(ev);
    if (it == events_.end())
      return nullptr;
    hipEvent_t e = it->second;
    events_.erase(it);
    return e;
  }

  int device_;
  std::vector<hipStream_t> streams_;
  std::mutex mu_;
  std::map<reloc::EventHandle, hipEvent_t> events_;
  reloc::EventHandle next_ = 1;
  bool failed_ = false;
  std::string error_;
};

void setErr(char *err, size_t cap, const std::string &msg) {
  if (err && cap) {
    std::strncpy(err, msg.c_str(), cap - 1);
    err[cap - 1] = 0;
  }
}

reloc::BufferView denseView(const void *p, size_t bytes, const std::vector<int64_t> &extents,
                            uint32_t elementSize, bool device, int ordinal) {
  reloc::BufferView v;
  v.base = reinterpret_cast<uintptr_t>(p);
  v.capacityBytes = bytes;
  v.offsetBytes = 0;
  v.extents = extents;
  v.strides.assign(extents.size(), 1);
  for (size_t k = extents.size(); k-- > 1;)
    v.strides[k - 1] = v.strides[k] * extents[k];
  v.elementSize = elementSize;
  v.kind = device ? reloc::MemoryKind::Cuda : reloc::MemoryKind::Host;
  v.device = device ? ordinal : -1;
  return v;
}

struct RefCpuH2d {
  bool typed = false;
  reloc::TypedBoundPlan typedPlan;
  reloc::BoundPlan layoutPlan;
  std::unique_ptr<reloc::GatherPool> pool;
  std::unique_ptr<HipCopyBackend> backend;
  int device = 0;
  int buffers = 2;
};

} // namespace

extern "C" {

// Decode + bind a typed (v1) or layout (v0) plan for the reference's CPU H2D
// path on `device` with `threads` transform workers, `buffers` pinned slots
// and `queues` copy streams. Parameters as ref_typed_prepare takes them.
void *ref_cpu_h2d_prepare(const uint8_t *blob, size_t n, const char **symNames,
                          const int64_t *symVals, int nsym, const char **paramNames,
                          const int *paramKind, const int *paramBits, const int64_t *paramLen,
                          const void **paramData, const size_t *paramBytes, int nparam,
                          unsigned threads, int buffers, int queues, int device, char *err,
                          size_t cap) {
  reloc::SymbolMap symbols;
  for (int i = 0; i < nsym; ++i)
    symbols[symNames[i]] = symVals[i];
  auto h = std::make_unique<RefCpuH2d>();
  h->device = device;
  h->buffers = buffers;
  if (reloc::peekWireVersion(blob, n).value_or(0) == 1) {
    auto decoded = reloc::decodeTypedPlan(blob, n);
    if (auto *e = std::get_if<reloc::DecodeError>(&decoded)) {
      setErr(err, cap, "decode: " + e->message);
      return nullptr;
    }
    reloc::ParameterMap params;
    for (int i = 0; i < nparam; ++i) {
      reloc::ParameterValue v;
      v.elementType = reloc::ElementType{static_cast<reloc::ElementTypeKind>(paramKind[i]),
                                         static_cast<uint32_t>(paramBits[i])};
      if (paramLen[i] >= 0)
        v.extents.push_back(paramLen[i]);
      const auto *p = static_cast<const uint8_t *>(paramData[i]);
      v.bytes.assign(p, p + paramBytes[i]);
      params[paramNames[i]] = std::move(v);
    }
    auto bound = reloc::bindTyped(std::get<reloc::TypedRelocationPlan>(decoded), symbols, params);
    if (auto *e = std::get_if<reloc::BindError>(&bound)) {
      setErr(err, cap, "bind: " + e->message);
      return nullptr;
    }
    h->typed = true;
    h->typedPlan = std::get<reloc::TypedBoundPlan>(std::move(bound));
  } else {
    auto decoded = reloc::decodePlan(blob, n);
    if (auto *e = std::get_if<reloc::DecodeError>(&decoded)) {
      setErr(err, cap, "decode: " + e->message);
      return nullptr;
    }
    auto bound = reloc::bind(std::get<reloc::RelocationPlan>(decoded), symbols);
    if (auto *e = std::get_if<reloc::BindError>(&bound)) {
      setErr(err, cap, "bind: " + e->message);
      return nullptr;
    }
    h->layoutPlan = std::get<reloc::BoundPlan>(std::move(bound));
  }
  if (threads > 1)
    h->pool = std::make_unique<reloc::GatherPool>(threads);
  h->backend = std::make_unique<HipCopyBackend>(device, queues > 0 ? queues : 1);
  if (h->backend->failed()) {
    setErr(err, cap, "backend: " + h->backend->error());
    return nullptr;
  }
  return h.release();
}

// Result bytes the plan writes on the device.
int64_t ref_cpu_h2d_result_bytes(void *handle) {
  auto *h = static_cast<RefCpuH2d *>(handle);
  return h->typed ? h->typedPlan.destinationBytes : h->layoutPlan.totalBytes;
}

// One blocking call: dense host source (source extents) -> device destination
// of the result bytes. Typed plans take the cpu_reference row
// (Policy::OriginalCpu); layout plans the layout H2D pipeline. Returns 0 on
// success; 1 with the reference's "<code>: <message>" otherwise.
int ref_cpu_h2d_execute(void *handle, const void *src, size_t srcBytes, void *dst,
                        size_t dstBytes, char *err, size_t cap) {
  auto *h = static_cast<RefCpuH2d *>(handle);
  reloc::TransferOptions options;
  options.nBuffers = h->buffers;
  options.gather = h->pool.get();
  options.gatherThreads = 1;
  options.pinning = reloc::PinningPolicy::Pinned;
  if (h->typed) {
    const reloc::TypedBoundPlan &p = h->typedPlan;
    const auto source = denseView(src, srcBytes, p.sourceExtents, p.sourceType.bitwidth / 8, false, -1);
    const auto destination = denseView(dst, dstBytes, p.resultExtents, p.resultType.bitwidth / 8, true,
                                       h->device);
    reloc::dispatch::Options o;
    o.policy = reloc::dispatch::Policy::OriginalCpu;
    auto request = reloc::dispatch::prepareDispatch(
        p, source, destination, reloc::TransferDirection::HostToDevice, o);
    if (auto *e = std::get_if<reloc::TransferError>(&request)) {
      setErr(err, cap, e->code + ": " + e->message);
      return 1;
    }
    auto &r = std::get<reloc::dispatch::DispatchRequest>(request);
    if (auto e = reloc::dispatch::executeDispatch(r, *h->backend, options)) {
      setErr(err, cap, e->code + ": " + e->message);
      return 1;
    }
    return 0;
  }
  const reloc::BoundPlan &p = h->layoutPlan;
  int64_t elements = 1;
  for (int64_t e : p.extents)
    elements *= e;
  const auto source = denseView(src, srcBytes, {elements}, p.elementSize, false, -1);
  const auto destination = denseView(dst, dstBytes, {p.totalBytes / p.elementSize}, p.elementSize,
                                     true, h->device);
  auto request =
      reloc::validateTransfer(p, source, destination, reloc::TransferDirection::HostToDevice);
  if (auto *e = std::get_if<reloc::TransferError>(&request)) {
    setErr(err, cap, e->code + ": " + e->message);
    return 1;
  }
  auto &r = std::get<reloc::TransferRequest>(request);
  if (auto e = reloc::executeTransfer(r, *h->backend, options)) {
    setErr(err, cap, e->code + ": " + e->message);
    return 1;
  }
  return 0;
}

void ref_cpu_h2d_free(void *handle) { delete static_cast<RefCpuH2d *>(handle); }

} // extern "C"
