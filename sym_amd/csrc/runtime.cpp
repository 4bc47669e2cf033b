// runtime.cpp - the H2D pipeline on one MI355X.
//
// Role of the reference's CudaBackend + Pipeline + transformToDevice
// (libreloc/cuda/CudaBackend.cu:55-282, libreloc/src/Pipeline.cpp:163-232,
// libreloc/src/Dispatch.cpp:246-564), designed for this GPU:
//
//   * compact bytes cross PCIe: the wire is the SOURCE at boundary k (int8 /
//     fp16 as stored, or the source after leading narrowing casts applied by
//     the host while it stages), never the widened result;
//   * chunks follow the source-outer axis, so each chunk's wire bytes are one
//     contiguous range and the kernel for that chunk needs nothing else;
//   * two copy streams take alternate chunks: host workers fill pinned ring
//     slot i (event-gated reuse), hipMemcpyAsync moves it to the device wire
//     buffer, and the chunk's relayout kernel follows on the same stream
//     while the next chunk is in flight on the other one.
// A page-locked source skips the ring and is DMA'd in place.
#include "runtime.h"

#include <dlfcn.h>
#include <immintrin.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>

#include "../../include/relx.h"

namespace relx {

#define HIPCHECK(expr)                                                                      \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess)                                                                   \
      throw Error("backend_failure", std::string(#expr) + ": " + hipGetErrorString(e_));    \
  } while (0)

// ------------------------------------------------------------ staging

namespace {

__attribute__((target("avx2,f16c"))) void f32_to_f16_f16c(const float *s, uint16_t *d,
                                                          int64_t n) {
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    const __m256 x = _mm256_loadu_ps(s + i);
    _mm_storeu_si128(reinterpret_cast<__m128i *>(d + i),
                     _mm256_cvtps_ph(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
  }
  for (; i < n; ++i) {
    uint32_t b;
    std::memcpy(&b, s + i, 4);
    d[i] = f32_to_f16_bits(b);
  }
}

// Exact binary16 -> binary32, eight at a time. The conversion instruction
// quiets signalling NaNs while the reference keeps the payload as is, so a
// batch holding a NaN goes through the scalar widening instead.
__attribute__((target("avx2,f16c"))) void f16_to_f32_f16c(const uint16_t *s, uint32_t *d,
                                                          int64_t n) {
  int64_t i = 0;
  const __m128i exp = _mm_set1_epi16(0x7c00), mant = _mm_set1_epi16(0x03ff);
  for (; i + 8 <= n; i += 8) {
    const __m128i h = _mm_loadu_si128(reinterpret_cast<const __m128i *>(s + i));
    const __m128i is_nan = _mm_and_si128(_mm_cmpeq_epi16(_mm_and_si128(h, exp), exp),
                                         _mm_xor_si128(_mm_cmpeq_epi16(_mm_and_si128(h, mant),
                                                                       _mm_setzero_si128()),
                                                       _mm_set1_epi16(-1)));
    if (_mm_movemask_epi8(is_nan)) {
      for (int j = 0; j < 8; ++j)
        d[i + j] = f16_to_f32_bits(s[i + j]);
      continue;
    }
    _mm256_storeu_ps(reinterpret_cast<float *>(d + i), _mm256_cvtph_ps(h));
  }
  for (; i < n; ++i)
    d[i] = f16_to_f32_bits(s[i]);
}

bool have_f16c() {
  static const bool ok = __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx2");
  return ok;
}

// A copy into a staging slot with streaming (non-temporal) stores: the slot
// is read next by the DMA engine, not by this core, and the stores skip the
// read-for-ownership of every destination line that a plain copy pays.
// Measured on the box's host (Zen 5, 32 MiB L3), 8 threads: a 32 MiB chunk
// of a source that is not in cache 430 -> 334 us; 8 MiB equal; a 2 MiB
// cache-resident chunk 8.6 -> 11.3 us, so only long ranges take it.
__attribute__((target("avx2"))) void copy_streaming(uint8_t *d, const uint8_t *s, size_t n) {
  size_t i = 0;
  while (i < n && (reinterpret_cast<uintptr_t>(d + i) & 31))
    d[i] = s[i], ++i;
  for (; i + 128 <= n; i += 128) {
    const __m256i a = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i));
    const __m256i b = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i + 32));
    const __m256i c = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i + 64));
    const __m256i e = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i + 96));
    _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i), a);
    _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i + 32), b);
    _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i + 64), c);
    _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i + 96), e);
  }
  for (; i < n; ++i)
    d[i] = s[i];
  _mm_sfence(); // the streaming stores are visible before the slot's copy is issued
}

bool have_avx2() {
  static const bool ok = __builtin_cpu_supports("avx2");
  return ok;
}

#ifndef RELX_STREAMING_STAGE_BYTES
#define RELX_STREAMING_STAGE_BYTES (size_t{2} << 20)
#endif

} // namespace

void host_transform(const Prepared &p, uint32_t k, uint32_t src_width, const void *src,
                    void *dst, int64_t e0, int64_t e1) {
  const uint8_t *s = static_cast<const uint8_t *>(src);
  uint8_t *d = static_cast<uint8_t *>(dst);
  if (k == 0) {
    const size_t n = static_cast<size_t>(e1 - e0) * src_width;
    // a worker's range of at least RELX_STREAMING_STAGE_BYTES (a chunk of
    // 16 MiB and more over 8 workers) streams its stores
    if (n >= RELX_STREAMING_STAGE_BYTES && have_avx2())
      copy_streaming(d + e0 * src_width, s + e0 * src_width, n);
    else
      std::memcpy(d + e0 * src_width, s + e0 * src_width, n);
    return;
  }
  if (k == 1 && p.stages[0].op == kOpF32toF16 && have_f16c()) {
    f32_to_f16_f16c(reinterpret_cast<const float *>(s) + e0, reinterpret_cast<uint16_t *>(d) + e0,
                    e1 - e0);
    return;
  }
  if (k == 1 && p.stages[0].op == kOpF16toF32 && have_f16c()) {
    f16_to_f32_f16c(reinterpret_cast<const uint16_t *>(s) + e0, reinterpret_cast<uint32_t *>(d) + e0,
                    e1 - e0);
    return;
  }
  const uint32_t wout = p.stages[k - 1].out_width;
  for (int64_t i = e0; i < e1; ++i) {
    uint64_t x = 0;
    std::memcpy(&x, s + i * src_width, src_width);
    for (uint32_t j = 0; j < k; ++j)
      x = host_apply(p.stages[j], x, 0);
    std::memcpy(d + i * wout, &x, wout);
  }
}

// ------------------------------------------------------------ tracing

namespace {

struct Roctx {
  int (*push)(const char *) = nullptr;
  int (*pop)() = nullptr;
};

// The ROCTX entry points when RELX_TRACE=1 and the library opens; else none.
const Roctx &roctx() {
  static const Roctx r = [] {
    Roctx t;
    const char *env = std::getenv("RELX_TRACE");
    if (!env || std::strcmp(env, "1") != 0)
      return t;
    void *h = dlopen("librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_GLOBAL);
    if (!h)
      h = dlopen("/opt/rocm/lib/librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_GLOBAL);
    if (!h)
      return t;
    t.push = reinterpret_cast<int (*)(const char *)>(dlsym(h, "roctxRangePushA"));
    t.pop = reinterpret_cast<int (*)()>(dlsym(h, "roctxRangePop"));
    if (!t.push || !t.pop)
      t = Roctx{};
    return t;
  }();
  return r;
}

} // namespace

TraceRange::TraceRange(const char *name, int64_t index, const char *key) {
  const Roctx &r = roctx();
  if (!r.push)
    return;
  char buf[96];
  std::snprintf(buf, sizeof(buf), "%s %s=%lld", name, key, static_cast<long long>(index));
  r.push(buf);
  open_ = true;
}

TraceRange::~TraceRange() {
  if (open_)
    roctx().pop();
}

// ------------------------------------------------------------ handles

const DeviceProgram &BoundHandle::program(uint32_t k) {
  std::lock_guard<std::mutex> g(mu);
  auto it = programs.find(k);
  if (it == programs.end())
    it = programs.emplace(k, build_program(*bound, prep, k)).first;
  return *it->second;
}

BoundHandle::DevParams BoundHandle::device_params(int device, uint32_t k) {
  const DeviceProgram &dp = program(k);
  std::lock_guard<std::mutex> g(mu);
  auto key = std::make_pair(device, k);
  auto it = params.find(key);
  if (it != params.end())
    return it->second;
  DevParams d;
  HIPCHECK(hipMalloc(&d.pf, dp.pf.size() * sizeof(float)));
  HIPCHECK(hipMalloc(&d.pi, dp.pi.size() * sizeof(int32_t)));
  HIPCHECK(hipMemcpy(d.pf, dp.pf.data(), dp.pf.size() * sizeof(float), hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(d.pi, dp.pi.data(), dp.pi.size() * sizeof(int32_t), hipMemcpyHostToDevice));
  params.emplace(key, d);
  return d;
}

BoundHandle::~BoundHandle() {
  for (auto &kv : params) {
    int cur = 0;
    if (hipGetDevice(&cur) == hipSuccess && cur != kv.first.first)
      (void)hipSetDevice(kv.first.first);
    (void)hipFree(kv.second.pf);
    (void)hipFree(kv.second.pi);
    if (cur != kv.first.first)
      (void)hipSetDevice(cur);
  }
  for (auto &kv : dev_indices) {
    DeviceScope scope(kv.first);
    (void)hipFree(kv.second);
  }
}

} // namespace relx

// ================================================================ driver

namespace relx {

namespace {

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess)
      prev = -1;
    if (prev != dev)
      HIPCHECK(hipSetDevice(dev));
  }
  ~DeviceGuard() {
    int cur;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev)
      (void)hipSetDevice(prev);
  }
};

#ifndef RELX_ZERO_COPY_BYTES
#define RELX_ZERO_COPY_BYTES (1 << 20)
#endif
constexpr int kChunkEvents = 32; // device-to-host kernel events, reused round robin

// A call's status flag, which the element-wise kernels set (pinned host
// memory). A slot is cleared when a call takes it, kStatusSlots calls after
// its previous user, and read after the call's work has completed.
int32_t read_status(const int32_t *status) {
  return *static_cast<const volatile int32_t *>(status);
}

void clear_status(int32_t *status) { *static_cast<volatile int32_t *>(status) = 0; }

// `s` waits for the work enqueued so far on the other copy streams among
// the first `used` (chunk c goes to stream c mod the call's stream count).
void join_copy_streams(Context &ctx, hipStream_t s, int64_t used) {
  for (int i = 0; i < kCopyStreams && i < used; ++i) {
    if (ctx.copies[i] == s)
      continue;
    HIPCHECK(hipEventRecord(ctx.join_ev[i], ctx.copies[i]));
    HIPCHECK(hipStreamWaitEvent(s, ctx.join_ev[i], 0));
  }
}

// The i-th pair of kernel timing events (created on first use, kept).
hipEvent_t *timing_pair(Context &ctx, size_t i) {
  while (ctx.time_ev.size() < 2 * (i + 1)) {
    hipEvent_t e;
    HIPCHECK(hipEventCreate(&e));
    ctx.time_ev.push_back(e);
  }
  return &ctx.time_ev[2 * i];
}

// Every copy stream waits for `ev`.
void copy_streams_wait(Context &ctx, hipEvent_t ev) {
  for (hipStream_t c : ctx.copies)
    HIPCHECK(hipStreamWaitEvent(c, ev, 0));
}

// Order after the caller's stream (relx_options.has_caller_stream, handle 0
// being the legacy null stream): the work enqueued on it so far may still
// produce a device source, read or write the destination, or fill a
// page-locked source. Only the call's operations that touch the caller's
// memory are ordered after it: kernels (they write the destination) and
// copies that read the caller's page-locked source. Copies out of the
// staging ring write only the library's own wire arena. When the caller's
// stream has no work left, nothing waits; else each of the call's streams
// waits on an event recorded on it, just before its first such operation,
// and not at all once that event has completed. On the MI355X a
// hipStreamWaitEvent on a pending event costs 10-15 us of host time (25 us
// on an event of the null stream), 0.15 us on a completed one: waiting on
// both copy streams up front put 20-50 us of host time before a call's
// first copy.
class CallerOrder {
public:
  CallerOrder(Context &ctx, const relx_options &opt) : ctx_(ctx) {
    if (!opt.has_caller_stream)
      return;
    hipStream_t caller = reinterpret_cast<hipStream_t>(opt.caller_stream);
    const hipError_t q = hipStreamQuery(caller);
    if (q == hipSuccess)
      return; // every earlier operation of the caller's stream has completed
    if (q != hipErrorNotReady)
      HIPCHECK(q);
    HIPCHECK(hipEventRecord(ctx.start_ev, caller));
    pending_ = true;
  }
  // Before an operation on `s` that touches the caller's memory.
  void before(hipStream_t s) {
    if (!pending_)
      return;
    for (int i = 0; i < kCopyStreams; ++i)
      if (ctx_.copies[i] == s && waited_[i])
        return;
    const hipError_t q = hipEventQuery(ctx_.start_ev);
    if (q == hipSuccess) {
      pending_ = false;
      return;
    }
    if (q != hipErrorNotReady)
      HIPCHECK(q);
    HIPCHECK(hipStreamWaitEvent(s, ctx_.start_ev, 0));
    for (int i = 0; i < kCopyStreams; ++i)
      if (ctx_.copies[i] == s)
        waited_[i] = true;
  }

private:
  Context &ctx_;
  bool pending_ = false;
  bool waited_[kCopyStreams] = {};
};

void ensure_wire(Context &ctx, size_t bytes) {
  if (ctx.wire_cap >= bytes)
    return;
  if (ctx.wire) {
    for (hipStream_t c : ctx.copies)
      HIPCHECK(hipStreamSynchronize(c));
    HIPCHECK(hipStreamSynchronize(ctx.compute));
    HIPCHECK(hipFree(ctx.wire));
    ctx.wire = nullptr;
    ctx.wire_cap = 0;
  }
  const size_t round = size_t{2} << 20;
  const size_t cap = (bytes + round - 1) / round * round;
  HIPCHECK(hipMalloc(&ctx.wire, cap));
  ctx.wire_cap = cap;
}

// The device copy of program k's parameter tables: the context's copy of
// these contents when it holds one, else a new entry when the cache has room,
// else the handle's own copy. Call with ctx.mu held and ctx.device current.
BoundHandle::DevParams context_params(Context &ctx, BoundHandle &h, uint32_t k) {
  const DeviceProgram &dp = h.program(k);
  const size_t fb = dp.pf.size() * sizeof(float), ib = dp.pi.size() * sizeof(int32_t);
  std::string key(sizeof(fb), '\0'); // the float bytes' length, then both tables
  std::memcpy(&key[0], &fb, sizeof(fb));
  key.append(reinterpret_cast<const char *>(dp.pf.data()), fb);
  key.append(reinterpret_cast<const char *>(dp.pi.data()), ib);
  auto it = ctx.param_cache.find(key);
  if (it != ctx.param_cache.end())
    return it->second;
  const size_t ioff = (fb + 255) / 256 * 256, bytes = ioff + ib;
  if (ctx.param_cache.size() >= kParamCacheEntries ||
      bytes > kParamCacheBytes - std::min(kParamCacheBytes, ctx.param_cache_bytes))
    return h.device_params(ctx.device, k);
  std::vector<uint8_t> host(bytes, 0);
  std::memcpy(host.data(), dp.pf.data(), fb);
  std::memcpy(host.data() + ioff, dp.pi.data(), ib);
  void *d = nullptr;
  HIPCHECK(hipMalloc(&d, bytes));
  const hipError_t e = hipMemcpy(d, host.data(), bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    HIPCHECK(e);
  }
  BoundHandle::DevParams par{static_cast<float *>(d),
                             reinterpret_cast<int32_t *>(static_cast<uint8_t *>(d) + ioff)};
  ctx.param_cache.emplace(std::move(key), par);
  ctx.param_cache_bytes += bytes;
  return par;
}

} // namespace

// Scratch kept between calls is bounded by ctx.max_retained (negative: no
// bound): once every call on the context has completed, the staging ring and
// the wire arena are released, the larger first, until what is kept fits.
// The next call that needs them allocates them again (reference
// dispatch::Resources: oversize scratch is released after completion,
// libreloc/include/reloc/DispatchResources.h:57-61,
// libreloc/src/DispatchResources.cpp:120-128,225).
void trim_retained(Context &ctx) {
  if (ctx.max_retained < 0 || ctx.unsynced)
    return;
  const size_t limit = static_cast<size_t>(ctx.max_retained);
  for (;;) {
    const size_t ring = ctx.slots.size() * ctx.slot_bytes;
    if (ring + ctx.wire_cap <= limit)
      return;
    if (ring >= ctx.wire_cap) {
      for (hipEvent_t e : ctx.slot_ev)
        HIPCHECK(hipEventSynchronize(e));
      for (void *s : ctx.slots)
        HIPCHECK(hipHostFree(s));
      for (hipEvent_t e : ctx.slot_ev)
        HIPCHECK(hipEventDestroy(e));
      ctx.slots.clear();
      ctx.slot_ev.clear();
      ctx.slot_pending.clear();
      ctx.slot_bytes = 0;
    } else {
      HIPCHECK(hipFree(ctx.wire));
      ctx.wire = nullptr;
      ctx.wire_cap = 0;
    }
  }
}

namespace {

constexpr unsigned kStagingThreads = 8, kGatherThreads = 12;

// The staging pool: exactly `need` threads when the caller gave a count,
// else at least `need` (a pool grown for an indexed gather is kept, and
// jobs that want fewer workers cap their ranges).
void ensure_workers(Context &ctx, unsigned need, bool exact) {
  if (ctx.workers && (exact ? ctx.worker_threads == need : ctx.worker_threads >= need))
    return;
  ctx.workers = std::make_unique<Workers>(need);
  ctx.worker_threads = need;
}

// The staging ring holds at least `n` slots of at least `slot_bytes`; true
// when this call allocated it (false: the ring kept from earlier calls fits).
// A new ring has exactly `n` slots: a call that stages one chunk gets one
// (reference: min(nBuffers, chunks) slots, libreloc/src/Dispatch.cpp:
// 524-531).
bool ensure_ring(Context &ctx, int n, size_t slot_bytes) {
  if (static_cast<int>(ctx.slots.size()) >= n && ctx.slot_bytes >= slot_bytes)
    return false;
  // drain users of the old ring before freeing it
  for (hipEvent_t e : ctx.slot_ev)
    HIPCHECK(hipEventSynchronize(e));
  for (void *s : ctx.slots)
    HIPCHECK(hipHostFree(s));
  for (hipEvent_t e : ctx.slot_ev)
    HIPCHECK(hipEventDestroy(e));
  ctx.slots.clear();
  ctx.slot_ev.clear();
  const size_t round = size_t{1} << 20;
  ctx.slot_bytes = (slot_bytes + round - 1) / round * round;
  const int want = std::max<int>(n, 1);
  for (int i = 0; i < want; ++i) {
    void *p = nullptr;
    HIPCHECK(hipHostMalloc(&p, ctx.slot_bytes, hipHostMallocDefault));
    ctx.slots.push_back(p);
    hipEvent_t e;
    HIPCHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    HIPCHECK(hipEventRecord(e, ctx.copies[0])); // a recorded, completed state
    ctx.slot_ev.push_back(e);
  }
  ctx.slot_pending.assign(ctx.slots.size(), false);
  return true;
}

// Copy streams a call spreads its chunks over: relx_options.n_streams 1
// keeps every copy and kernel on one stream; 0 (default) and 2 or more use
// the context's kCopyStreams.
int call_streams(const relx_options &opt) {
  if (opt.n_streams < 0)
    throw Error("invalid_options", "n_streams must be >= 0 (0: the default)");
  return opt.n_streams == 1 ? 1 : kCopyStreams;
}

// The host writes a staging slot only after the device work that last read
// it: the slot's event is waited for when one was recorded since the slot
// was last known idle.
void slot_acquire(Context &ctx, int slot) {
  const size_t i = static_cast<size_t>(slot);
  if (ctx.slot_pending[i]) {
    HIPCHECK(hipEventSynchronize(ctx.slot_ev[i]));
    ctx.slot_pending[i] = false;
  }
}

// Once the work that reads the slot is enqueued on `s`. `track` is false
// when no later chunk of a blocking call reuses the slot: the call's final
// synchronization proves every read of the slot done before the host can
// write it again, so no event is recorded (two runtime calls fewer per
// chunk, about 4 us of a small call).
void slot_release(Context &ctx, int slot, hipStream_t s, bool track) {
  if (!track)
    return;
  const size_t i = static_cast<size_t>(slot);
  HIPCHECK(hipEventRecord(ctx.slot_ev[i], s));
  ctx.slot_pending[i] = true;
}

// A call from another thread than the previous call's, after that call
// completed: it synchronizes with the previous call's end (done_ev, already
// complete) before it writes any staging slot, so that its host writes are
// ordered after every device read of the earlier calls through the runtime,
// not only through the context's lock. Calls from one thread are ordered by
// program order; after a call that returned early the slots' events order
// them.
void order_after_previous_thread(Context &ctx) {
  const std::thread::id self = std::this_thread::get_id();
  if (ctx.last_thread == self)
    return;
  if (ctx.last_thread != std::thread::id() && !ctx.unsynced)
    HIPCHECK(hipEventSynchronize(ctx.done_ev));
  ctx.last_thread = self;
}

bool probe_pinned(const void *p) {
  hipPointerAttribute_t attr;
  const hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError(); // pageable memory: clear the probe's error
    return false;
  }
  return attr.type == hipMemoryTypeHost;
}

// Leading stages the host applies while staging: per-tensor stages that do
// not widen the element (so the wire shrinks or stays), stopping at the
// first per-channel or widening stage.
} // namespace

uint32_t auto_host_stages(const BoundHandle &h) {
  if (!h.bound->typed)
    return 0;
  uint32_t k = 0;
  uint32_t width = h.bound->source_type.width();
  for (const HostStage &s : h.prep.stages) {
    if (s.mode != kChanNone || s.out_width >= width)
      break;
    width = s.out_width;
    ++k;
  }
  return k;
}

namespace {

struct Member {
  BoundHandle *h;
  const uint8_t *src;
  size_t src_bytes;
  uint8_t *dst;
  size_t dst_bytes;
  relx_report *report;
  uint32_t k;
  const DeviceProgram *dp;
  bool direct;
  size_t wire_off;
  bool table; // indexed: the table crosses PCIe and the device gathers the rows
  int64_t arena_bytes; // wire arena bytes of this member
  bool zero_copy = false; // one small chunk: the kernels read its ring slot
};

// The device memory an allocation-free call uses in place of the context's
// wire arena and the bound plan's parameter tables: regions of the
// library's static scratch array, and the host tables uploaded into it.
struct StaticScratch {
  uint8_t *wire;
  size_t wire_cap;
  float *pf;
  int32_t *pi;
  const std::vector<float> *host_pf;
  const std::vector<int32_t> *host_pi;
  hipEvent_t last; // the end of the device's previous static call (StaticDevice::last)
};

} // namespace

void execute(Context &ctx, std::vector<Member> &members, const relx_options &opt,
             relx_report *total, Completion *comp, const StaticScratch *sc = nullptr);

} // namespace relx

// The functions below are reached through capi.cpp.
namespace relx {

void execute_members(Context &ctx, int n, BoundHandle *const *bounds, const void *const *srcs,
                     const size_t *src_bytes, void *const *dsts, const size_t *dst_bytes,
                     const relx_options &opt, relx_report *reports, relx_report *total,
                     Completion *comp) {
  TraceRange call_range("relx.h2d.call", ctx.calls, "call");
  DeviceGuard guard(ctx.device);
  std::vector<Member> ms;
  size_t wire_total = 0;
  const int hs = opt.host_stages;
  for (int i = 0; i < n; ++i) {
    BoundHandle *h = bounds[i];
    Member m{h, static_cast<const uint8_t *>(srcs[i]), src_bytes[i],
             static_cast<uint8_t *>(dsts[i]), dst_bytes[i], reports ? &reports[i] : nullptr, 0,
             nullptr, false, 0, false, 0};
    const bool indexed = h->bound->indexed;
    // An indexed plan's rows are scattered over the table: always staged.
    const bool pinned = !indexed && (opt.source_pinned > 0 ||
                                     (opt.source_pinned < 0 && probe_pinned(m.src)));
    const uint32_t nst = static_cast<uint32_t>(h->prep.stages.size());
    // Automatic: the leading narrowing stages, from a pinned source too.
    // Staging C2 (f32 -> f16) from a pinned source takes 0.22 ms against
    // 0.36 ms for the direct DMA of the f32 source (32 images; 0.85 against
    // 1.40 ms for 128): the host casts faster than PCIe moves the bytes it
    // saves. A source with no such stage is sent by direct DMA.
    if (hs < 0)
      m.k = auto_host_stages(*h);
    else
      m.k = static_cast<uint32_t>(std::min<int>(hs, static_cast<int>(nst)));
    for (uint32_t j = 0; j < m.k; ++j)
      if (h->prep.stages[j].mode != kChanNone)
        throw Error("invalid_options", "host stages must be per-tensor stages");
    m.dp = &h->program(m.k);
    m.direct = pinned && m.k == 0;
    const Bound &b = *h->bound;
    m.arena_bytes = m.dp->wire_bytes;
    if (indexed && hs < 0 && table_upload_pays(b, m.dp->wire_bytes) &&
        reinterpret_cast<uintptr_t>(m.dst) % b.result_type.width() == 0) {
      m.table = true;
      m.k = 0;
      m.dp = &h->program(0);
      m.direct = opt.source_pinned > 0 || (opt.source_pinned < 0 && probe_pinned(m.src));
      m.arena_bytes = b.table_bytes;
    }
    const int64_t need_src = indexed ? b.table_bytes
                             : b.typed ? b.source_bytes
                                       : m.dp->wire_elems * static_cast<int64_t>(b.layout.element_size);
    if (static_cast<int64_t>(m.src_bytes) < need_src)
      throw Error("insufficient_capacity", "source holds " + std::to_string(m.src_bytes) +
                                               " bytes, the plan reads " + std::to_string(need_src));
    const int64_t need_dst = m.dp->dst_elems * m.dp->base.wout;
    if (static_cast<int64_t>(m.dst_bytes) < need_dst)
      throw Error("insufficient_capacity", "destination holds " + std::to_string(m.dst_bytes) +
                                               " bytes, the plan writes " + std::to_string(need_dst));
    if (!m.src || !m.dst)
      throw Error("invalid_view", "null source or destination");
    m.wire_off = wire_total;
    wire_total += (static_cast<size_t>(m.arena_bytes) + 255) / 256 * 256;
    ms.push_back(m);
  }
  execute(ctx, ms, opt, total, comp);
}

// The allocation-free upload: the pipeline above with the wire staged in the
// library's static device scratch and the parameter tables uploaded into it,
// from a page-locked source by direct DMA (no ring), with no worker pool and
// no timing events. It allocates no device or pinned host memory.
void execute_static(Context &ctx, BoundHandle &h, const void *src, size_t src_bytes, void *dst,
                    size_t dst_bytes, const relx_options &opt, relx_report *report) {
  DeviceGuard guard(ctx.device);
  if (!ctx.stat || !ctx.param_stage)
    throw Error("backend_failure", "the static scratch is not mapped on this context's device");
  // one static call at a time on the device, whatever the context
  std::lock_guard<std::mutex> serial(ctx.stat->mu);
  const Bound &b = *h.bound;
  if (b.indexed)
    throw Error("plan_mismatch", "the allocation-free upload takes layout and typed plans; "
                                 "indexed plans gather host rows through the staging ring");
  if (opt.host_stages > 0)
    throw Error("invalid_options", "the allocation-free upload applies no host stages: "
                                   "the source crosses as it is");
  if (!src || !dst)
    throw Error("invalid_view", "null source or destination");
  const bool pinned = opt.source_pinned > 0 || (opt.source_pinned < 0 && probe_pinned(src));
  if (!pinned)
    throw Error("invalid_options", "the allocation-free upload needs a page-locked source: "
                                   "it has no staging ring to allocate");
  const DeviceProgram &dp = h.program(0);
  const int64_t need_src = b.typed ? b.source_bytes : dp.wire_elems * b.layout.element_size;
  if (static_cast<int64_t>(src_bytes) < need_src)
    throw Error("insufficient_capacity", "source holds " + std::to_string(src_bytes) +
                                             " bytes, the plan reads " + std::to_string(need_src));
  const int64_t need_dst = dp.dst_elems * dp.base.wout;
  if (static_cast<int64_t>(dst_bytes) < need_dst)
    throw Error("insufficient_capacity", "destination holds " + std::to_string(dst_bytes) +
                                             " bytes, the plan writes " + std::to_string(need_dst));
  if (static_cast<size_t>(dp.wire_bytes) > kScratchWireBytes)
    throw Error("insufficient_capacity",
                "the plan's wire is " + std::to_string(dp.wire_bytes) +
                    " bytes; the allocation-free upload stages at most " +
                    std::to_string(kScratchWireBytes) + " bytes");
  if (dp.pf.size() * sizeof(float) > kParamStageHalf ||
      dp.pi.size() * sizeof(int32_t) > kParamStageHalf)
    throw Error("insufficient_capacity", "the plan's parameter tables exceed the static scratch's " +
                                             std::to_string(kParamStageHalf) + "-byte tables");
  if (ctx.unsynced) { // an earlier call may still read the pinned parameter staging
    HIPCHECK(hipEventSynchronize(ctx.done_ev));
    ctx.unsynced = false;
  }
  std::vector<Member> ms{Member{&h, static_cast<const uint8_t *>(src), src_bytes,
                                static_cast<uint8_t *>(dst), dst_bytes, report, 0, &dp, true, 0,
                                false, dp.wire_bytes}};
  uint8_t *tables = ctx.stat->addr + kScratchWireBytes;
  const StaticScratch sc{ctx.stat->addr, kScratchWireBytes, reinterpret_cast<float *>(tables),
                         reinterpret_cast<int32_t *>(tables + kParamStageHalf), &dp.pf, &dp.pi,
                         ctx.stat->last};
  execute(ctx, ms, opt, nullptr, nullptr, &sc);
}

void execute(Context &ctx, std::vector<Member> &ms, const relx_options &opt,
             relx_report *total, Completion *comp, const StaticScratch *sc) {
  order_after_previous_thread(ctx); // before any host access to the ring or the arena
  size_t wire_total = 0;
  for (const Member &m : ms)
    wire_total = std::max(wire_total, m.wire_off + static_cast<size_t>(m.arena_bytes));
  if (!sc)
    ensure_wire(ctx, wire_total);
  else if (wire_total > sc->wire_cap)
    throw Error("insufficient_capacity", "the wire needs " + std::to_string(wire_total) +
                                             " bytes; the static scratch holds " +
                                             std::to_string(sc->wire_cap));

  // Chunk plan per member: units of the chunk axis per chunk (a table upload:
  // byte ranges of the table, multiples of 256 bytes).
  size_t max_slot = 0;
  std::vector<ChunkPlan> plans;
  // Ring slots. With the chunks left to the library (chunk_bytes unset) the
  // depth is the library's too, n_buffers counting as a minimum: a ring of
  // two slots stages chunk j only once the copy of chunk j - 2 has landed,
  // and the copy engines idle whenever a staging outlasts the other slot's
  // copy. Pageable sources, p50 of raw calls, two slots -> three: C1 0.83-0.88
  // -> 0.91-0.92 of the PCIe ceiling, C2 0.71-0.72 -> 0.76-0.77, C5 [8,1024]
  // 0.83-0.88 -> 0.92, [8,4096] 0.91-0.92 -> 0.94-0.95, [64,4096] 0.96 ->
  // 0.99. A caller's chunk_bytes keeps the slots it asks for.
  const int nslots = opt.n_buffers <= 0 ? 3
                     : opt.chunk_bytes > 0 ? opt.n_buffers
                                           : std::max(opt.n_buffers, 3);
  for (Member &m : ms) {
    const DeviceProgram &dp = *m.dp;
    ChunkPlan p{};
    if (m.table) {
      const int64_t tb = m.h->bound->table_bytes;
      const int64_t want =
          opt.chunk_bytes > 0 ? opt.chunk_bytes : default_chunk_bytes(tb, true, m.direct);
      p.units = tb;
      p.per_chunk = std::min(tb, std::max<int64_t>(256, want / 256 * 256));
      p.unit_wire = p.unit_src = 1;
    } else {
      p = chunk_plan(dp, source_width(*m.h->bound), opt.chunk_bytes, m.direct);
      // A staged wire of at most RELX_ZERO_COPY_BYTES that crosses as one
      // chunk: the kernels read its ring slot over PCIe, with no copy ahead
      // of them. Kernels read only the library's own page-locked memory,
      // never the caller's (a pinned source keeps its direct copy, which
      // measured faster than staging it for a zero-copy read).
      m.zero_copy = !sc && !m.direct && p.units <= p.per_chunk &&
                    dp.wire_bytes <= static_cast<int64_t>(RELX_ZERO_COPY_BYTES);
    }
    if (!m.direct)
      max_slot = std::max(max_slot, static_cast<size_t>(p.per_chunk * p.unit_wire));
    plans.push_back(p);
  }
  int64_t total_chunks = 0, staged = 0; // every chunk, the staged ones
  for (size_t i = 0; i < ms.size(); ++i) {
    const int64_t n = (plans[i].units + plans[i].per_chunk - 1) / plans[i].per_chunk;
    total_chunks += n;
    if (!ms[i].direct)
      staged += n;
  }
  const int ns = call_streams(opt);
  const bool two_streams = total_chunks > 1 && ns > 1; // else one copy stream does everything
  if (max_slot && sc)
    throw Error("invalid_options", "an allocation-free call has no staging ring");
  const bool ring_new =
      max_slot && ensure_ring(ctx, static_cast<int>(std::min<int64_t>(nslots, staged)), max_slot);
  // A slot's event is needed when the call returns before its work
  // completes, or when a later chunk of this call reuses the slot (staged
  // chunk j takes slot j mod ring size).
  const bool early = comp != nullptr || opt.no_wait != 0;
  const int64_t nring = static_cast<int64_t>(ctx.slots.size());
  int64_t staged_no = 0; // staged chunks so far
  auto next_track = [&] { return early || staged_no++ + nring < staged; };
  // Staging workers: the caller's count for every job when it gives one;
  // else 8, and 12 for the host row gathers of indexed plans, whose random
  // rows want more reads in flight (ix f32 -> f16, 64 Ki rows of 4 KiB:
  // 2.55 ms with 12 against 2.8-3.5 ms with 8).
  const bool exact = opt.gather_threads > 0;
  const unsigned parts = exact ? static_cast<unsigned>(opt.gather_threads) : kStagingThreads;
  const unsigned gparts = exact ? parts : kGatherThreads;
  bool gathers = false;
  for (const Member &m : ms)
    gathers = gathers || (m.h->bound->indexed && !m.table && !m.direct);
  if (!sc)
    ensure_workers(ctx, gathers ? std::max(parts, gparts) : parts, exact);

  // Each chunk's kernel runs on the stream that copied the chunk (a kernel
  // behind a copy on one stream starts about 10 us sooner than one ordered
  // by an event from another stream); the copy streams join at the end.
  if (ctx.unsynced) // the previous call may still read the wire arena
    copy_streams_wait(ctx, ctx.done_ev);
  // The caller's stream orders the call's kernels and direct copies
  // (libreloc/src/Dispatch.cpp:1995, libreloc/cuda/CudaBackend.cu:190-208).
  const bool ordered = opt.has_caller_stream != 0;
  hipStream_t caller = reinterpret_cast<hipStream_t>(opt.caller_stream);
  CallerOrder order(ctx, opt);
  bool any_generic = false;
  for (const Member &m : ms)
    any_generic = any_generic || m.dp->family == kFamGeneric;
  int32_t *status = ctx.status + (ctx.status_next++ % kStatusSlots);
  if (any_generic)
    clear_status(status);
  if (sc) {
    // The scratch is free once the device's previous static call, from any
    // context, has completed: the table copies wait for its end, and the
    // other copy stream waits for them below.
    const hipError_t q = hipEventQuery(sc->last);
    if (q == hipErrorNotReady)
      HIPCHECK(hipStreamWaitEvent(ctx.copies[0], sc->last, 0));
    else if (q != hipSuccess)
      HIPCHECK(q);
    // The parameter tables go to the scratch through the context's pinned
    // staging (a DMA, no runtime staging), ahead of every chunk's kernel.
    const size_t fb = sc->host_pf->size() * sizeof(float), ib = sc->host_pi->size() * sizeof(int32_t);
    std::memcpy(ctx.param_stage, sc->host_pf->data(), fb);
    std::memcpy(ctx.param_stage + kParamStageHalf, sc->host_pi->data(), ib);
    HIPCHECK(hipMemcpyAsync(sc->pf, ctx.param_stage, fb, hipMemcpyHostToDevice, ctx.copies[0]));
    HIPCHECK(hipMemcpyAsync(sc->pi, ctx.param_stage + kParamStageHalf, ib, hipMemcpyHostToDevice,
                            ctx.copies[0]));
    HIPCHECK(hipEventRecord(ctx.join_ev[0], ctx.copies[0]));
    for (int i = 1; i < kCopyStreams; ++i)
      HIPCHECK(hipStreamWaitEvent(ctx.copies[i], ctx.join_ev[0], 0));
  }

  int slot = 0;
  int64_t nchunk = 0; // chunks of every member so far: picks the copy stream
  relx_report sum{};
  // Kernel timing covers blocking calls, whose events are read at the end.
  const bool timing = ctx.time_kernels && !comp && !opt.no_wait && !sc;
  size_t tpairs = 0;
  for (size_t mi = 0; mi < ms.size(); ++mi) {
    Member &m = ms[mi];
    const DeviceProgram &dp = *m.dp;
    const ChunkPlan &p = plans[mi];
    const BoundHandle::DevParams par =
        sc ? BoundHandle::DevParams{sc->pf, sc->pi} : context_params(ctx, *m.h, m.k);
    const uint32_t sw = m.h->bound->typed ? m.h->bound->source_type.width()
                                          : m.h->bound->layout.element_size;
    uint8_t *wire = (sc ? sc->wire : ctx.wire) + m.wire_off;
    int64_t chunks = 0, launches = 0;
    if (m.table) {
      // The table crosses as it is (byte chunks); the gather reads rows from
      // every chunk, so it waits for both copy streams.
      const Bound &bd = *m.h->bound;
      (void)m.h->device_indices(ctx.device); // uploaded before the copies start
      hipStream_t cs = ctx.copies[0];
      for (int64_t b0 = 0; b0 < p.units; b0 += p.per_chunk) {
        const int64_t n = std::min(p.per_chunk, p.units - b0);
        cs = ctx.copy_stream(nchunk++, ns);
        if (m.direct) {
          order.before(cs);
          HIPCHECK(hipMemcpyAsync(wire + b0, m.src + b0, static_cast<size_t>(n),
                                  hipMemcpyHostToDevice, cs));
        } else {
          uint8_t *s = static_cast<uint8_t *>(ctx.slots[static_cast<size_t>(slot)]);
          slot_acquire(ctx, slot);
          const uint8_t *from = m.src + b0;
          ctx.workers->parallel_for(n, int64_t{1} << 18, [&](int64_t x, int64_t y) {
            std::memcpy(s + x, from + x, static_cast<size_t>(y - x));
          }, parts);
          HIPCHECK(hipMemcpyAsync(wire + b0, s, static_cast<size_t>(n), hipMemcpyHostToDevice, cs));
          slot_release(ctx, slot, cs, next_track());
          slot = (slot + 1) % static_cast<int>(ctx.slots.size());
        }
        ++chunks;
      }
      if (chunks > 1 && ns > 1)
        join_copy_streams(ctx, cs, nchunk);
      order.before(cs);
      launches = index_select_device(ctx, *m.h, wire, static_cast<size_t>(bd.table_bytes), m.dst,
                                     m.dst_bytes, cs);
    }
    const KernelBatches kb = kernel_batches(p);
    int zc_slot = -1; // the ring slot a zero-copy member's kernels read
    bool zc_track = false;
    int64_t kb0 = 0; // first unit of the kernel batch being gathered
    for (int64_t v0 = 0; v0 < (m.table ? 0 : p.units); v0 += p.per_chunk) {
      const int64_t v1 = std::min(p.units, v0 + p.per_chunk);
      const int64_t woff = v0 * p.unit_wire, wbytes = (v1 - v0) * p.unit_wire;
      const int64_t chunk_no = nchunk;
      hipStream_t cs = ctx.copy_stream(nchunk++, ns);
      const uint8_t *kwire = wire; // what the batch's kernels read
      if (m.direct) {
        TraceRange tr("relx.h2d.submit", chunk_no);
        order.before(cs);
        HIPCHECK(hipMemcpyAsync(wire + woff, m.src + woff, static_cast<size_t>(wbytes),
                                hipMemcpyHostToDevice, cs));
      } else {
        uint8_t *s = static_cast<uint8_t *>(ctx.slots[static_cast<size_t>(slot)]);
        {
          TraceRange tr("relx.h2d.slot_wait", chunk_no);
          slot_acquire(ctx, slot);
        }
        TraceRange tr("relx.h2d.stage", chunk_no);
        const int64_t e0 = v0 * (p.unit_src / sw), e1 = v1 * (p.unit_src / sw);
        const int64_t ne = e1 - e0;
        const uint8_t *src_base = m.src + e0 * sw;
        const uint32_t k = m.k;
        const Prepared &prep = m.h->prep;
        const Bound &bd = *m.h->bound;
        // each worker converts a contiguous element range into the slot
        if (bd.indexed) {
          const int64_t wout = dp.base.win; // wire element bytes at boundary k
          ctx.workers->parallel_for(ne, int64_t{1} << 16, [&](int64_t a, int64_t b) {
            host_gather(bd, prep, k, m.src, s + a * wout, e0 + a, e0 + b);
          }, gparts);
        } else {
          ctx.workers->parallel_for(ne, int64_t{1} << 16, [&](int64_t a, int64_t b) {
            host_transform(prep, k, sw, src_base, s, a, b);
          }, parts);
        }
        if (m.zero_copy) {
          kwire = s; // the slot is released after the kernels that read it
          zc_slot = slot;
          zc_track = next_track();
        } else {
          HIPCHECK(hipMemcpyAsync(wire + woff, s, static_cast<size_t>(wbytes),
                                  hipMemcpyHostToDevice, cs));
          slot_release(ctx, slot, cs, next_track());
        }
        slot = (slot + 1) % static_cast<int>(ctx.slots.size());
      }
      ++chunks;
      if (v1 < kb.end(kb0))
        continue; // the kernel batch takes more chunks
      // The batch's launches follow this chunk's copy on its stream, and the
      // other copy stream's copies of the batch through an event.
      if (kb0 < v0 && two_streams)
        join_copy_streams(ctx, cs, nchunk);
      // Timing events bracket the batch's launches on the stream they run
      // on; the first completes when the batch's copies have landed.
      order.before(cs);
      hipEvent_t *tev = timing ? timing_pair(ctx, tpairs++) : nullptr;
      if (tev)
        HIPCHECK(hipEventRecord(tev[0], cs));
      const int64_t nl = launch_program(dp, kb0, v1, kb0 == 0, v1 == p.units, kwire, m.dst,
                                        par.pf, par.pi, status, cs);
      if (zc_slot >= 0) {
        slot_release(ctx, zc_slot, cs, zc_track);
        zc_slot = -1;
      }
      if (tev) {
        HIPCHECK(hipEventRecord(tev[1], cs));
        ctx.kt.launches += nl;
      }
      launches += nl;
      kb0 = v1;
    }
    if (m.report) {
      relx_report &r = *m.report;
      std::memset(&r, 0, sizeof(r));
      const std::string impl = m.table  ? std::string("hip_table_gather")
                               : m.k == 0 ? std::string("hip_relayout")
                                          : "hip_relayout@" + std::to_string(m.k);
      std::snprintf(r.implementation, sizeof(r.implementation), "%s", impl.c_str());
      const Bound &b = *m.h->bound;
      r.source_bytes = b.indexed ? b.table_bytes : b.typed ? b.source_bytes : dp.wire_elems * sw;
      r.wire_bytes = m.arena_bytes;
      r.destination_bytes = dp.dst_elems * dp.base.wout;
      r.parameter_bytes = b.parameter_bytes;
      r.payload_bytes_transferred = m.arena_bytes;
      r.chunks = chunks;
      r.kernel_launches = launches;
      r.wire_boundary = static_cast<int>(m.k);
      r.direct_dma = m.direct ? 1 : 0;
      r.host_chunk_bytes = std::min(m.arena_bytes, p.per_chunk * p.unit_wire);
      r.host_buffers = m.direct ? 0 : std::min(nring, chunks);
      r.staging_bytes = staged ? nring * static_cast<int64_t>(ctx.slot_bytes) : 0;
      r.staging_slots = staged ? nring : 0;
      r.staging_reused = staged && !ring_new ? 1 : 0;
      r.copy_streams = static_cast<int>(std::min<int64_t>(ns, total_chunks));
      sum.source_bytes += r.source_bytes;
      sum.wire_bytes += r.wire_bytes;
      sum.destination_bytes += r.destination_bytes;
      sum.parameter_bytes += r.parameter_bytes;
      sum.payload_bytes_transferred += r.payload_bytes_transferred;
      sum.chunks += r.chunks;
      sum.kernel_launches += r.kernel_launches;
      sum.host_chunk_bytes = std::max(sum.host_chunk_bytes, r.host_chunk_bytes);
      sum.direct_dma = mi == 0 ? r.direct_dma : sum.direct_dma && r.direct_dma;
      sum.host_buffers = std::min(nring, staged);
      sum.staging_bytes = r.staging_bytes;
      sum.staging_slots = r.staging_slots;
      sum.staging_reused = r.staging_reused;
      sum.copy_streams = r.copy_streams;
    }
  }
  // join on the stream of the last chunk (the others are usually done)
  hipStream_t last = nchunk > 0 ? ctx.copy_stream(nchunk - 1, ns) : ctx.copies[0];
  if (two_streams)
    join_copy_streams(ctx, last, nchunk);
  HIPCHECK(hipEventRecord(ctx.done_ev, last));
  if (sc) // the next static call on the device writes the scratch after this
    HIPCHECK(hipEventRecord(sc->last, last));
  // A call that returns before its work completes orders the caller's
  // stream after it; a blocking call has completed when it returns, so
  // anything the caller enqueues next runs after it without a wait.
  if (ordered && early)
    HIPCHECK(hipStreamWaitEvent(caller, ctx.done_ev, 0));
  if (total) {
    std::snprintf(sum.implementation, sizeof(sum.implementation), "hip_relayout_group");
    *total = sum;
  }
  if (comp) {
    HIPCHECK(hipEventRecord(comp->ev, last));
    comp->status = status;
    comp->generic = any_generic;
    ctx.unsynced = true;
    return;
  }
  if (opt.no_wait) {
    ctx.unsynced = true;
    return;
  }
  HIPCHECK(hipEventSynchronize(ctx.done_ev));
  ctx.unsynced = false;
  std::fill(ctx.slot_pending.begin(), ctx.slot_pending.end(), false); // every read is done
  if (!sc)
    trim_retained(ctx);
  if (timing) {
    for (size_t i = 0; i < tpairs; ++i) {
      float ms = 0.0f;
      HIPCHECK(hipEventElapsedTime(&ms, ctx.time_ev[2 * i], ctx.time_ev[2 * i + 1]));
      ctx.kt.ms += ms;
    }
    ctx.kt.chunks += static_cast<int64_t>(tpairs);
    ++ctx.kt.calls;
  }
  if (any_generic) {
    if (read_status(status))
      throw Error("channel_out_of_range", "a stage selected a channel outside its parameters");
  }
}

void completion_wait(Completion &c) {
  DeviceGuard guard(c.ctx->device);
  HIPCHECK(hipEventSynchronize(c.ev));
  completion_check(c);
}

// Once the completion's event has completed: the call's status flag.
void completion_check(Completion &c) {
  if (c.generic && !c.checked) {
    c.checked = true;
    if (read_status(c.status))
      throw Error("channel_out_of_range", "a stage selected a channel outside its parameters");
  }
}

// --------------------------------------------------------------- D2H

D2hPlan d2h_plan(const DeviceProgram &dp, int64_t chunk_bytes, bool pinned) {
  const KArgs &a = dp.base;
  const int64_t out_bytes = dp.dst_elems * a.wout;
  D2hPlan p{-1, 1, 1, 1, out_bytes, out_bytes};
  bool dense = true;
  int64_t run = 1;
  for (int k = a.rank - 1; k >= 0; --k) {
    dense = dense && a.ds[k] == run;
    run *= a.pext[k];
  }
  if (!dense || run != dp.dst_elems || a.rank < 1)
    return p;
  const int64_t want = chunk_bytes > 0 ? chunk_bytes : default_chunk_bytes(out_bytes, false, pinned);
  p.copy_bytes = std::min(out_bytes, want);
  // the outermost axis one coordinate of which fits a chunk; the axes before
  // it must accept single-coordinate boxes
  int64_t outer = 1;
  for (int j = 0; j < a.rank; ++j) {
    const int64_t al = axis_align(dp, j);
    const int64_t row = out_bytes / outer / a.pext[j];
    if (al <= 0)
      return p;
    if (row * al <= want || j == a.rank - 1) {
      if (a.pext[j] <= al && outer == 1)
        return p; // one chunk
      p.axis = j;
      p.outer = outer;
      p.units = a.pext[j];
      p.row = row;
      int64_t per = std::max<int64_t>(1, want / std::max<int64_t>(1, row));
      per = std::max<int64_t>(al, per / al * al);
      p.per = std::min(per, p.units);
      return p;
    }
    if (al != 1)
      return p; // a fixed coordinate would break the axis' alignment
    outer *= a.pext[j];
  }
  return p;
}

// Device -> host: the device runs the relayout and every stage, one
// destination-row chunk at a time, into the context's device result buffer;
// each chunk then crosses PCIe while the next chunk's kernel runs. A pinned
// destination takes the DMA directly; a pageable one goes through the pinned
// ring and the worker threads copy each slot out as soon as its copy lands.
void execute_d2h(Context &ctx, BoundHandle &h, const void *src, size_t src_bytes, void *dst,
                 size_t dst_bytes, const relx_options &opt, relx_report *report) {
  TraceRange call_range("relx.d2h.call", ctx.calls, "call");
  DeviceGuard guard(ctx.device);
  order_after_previous_thread(ctx);
  if (h.bound->indexed) // libreloc/src/Dispatch.cpp:196-201: indexed sources are host rows
    throw Error("plan_mismatch", "indexed source requires the prepared host row shape");
  const DeviceProgram &dp = h.program(0);
  const Bound &b = *h.bound;
  if (!src || !dst)
    throw Error("invalid_view", "null source or destination");
  if (static_cast<int64_t>(src_bytes) < dp.wire_bytes)
    throw Error("insufficient_capacity", "source holds " + std::to_string(src_bytes) +
                                             " bytes, the plan reads " +
                                             std::to_string(dp.wire_bytes));
  const int64_t out_bytes = dp.dst_elems * dp.base.wout;
  if (static_cast<int64_t>(dst_bytes) < out_bytes)
    throw Error("insufficient_capacity", "destination holds " + std::to_string(dst_bytes) +
                                             " bytes, the plan writes " +
                                             std::to_string(out_bytes));
  ensure_wire(ctx, static_cast<size_t>(out_bytes)); // the device result
  const bool pinned = opt.source_pinned > 0 || (opt.source_pinned < 0 && probe_pinned(dst));

  const D2hPlan plan = d2h_plan(dp, opt.chunk_bytes, pinned);
  const int axis = plan.axis;
  // without a chunk axis the kernel runs once and only the copies are chunked
  const int64_t units = axis < 0 ? (out_bytes + plan.copy_bytes - 1) / plan.copy_bytes : plan.units;
  const int64_t row = axis < 0 ? plan.copy_bytes : plan.row, per = axis < 0 ? 1 : plan.per;
  const KArgs &a = dp.base;
  const int64_t total_chunks = plan.outer * ((units + per - 1) / per);
  // ring slots, at most one per chunk: n_buffers, at least three when the
  // library picks the chunks (as for uploads)
  const int asked = opt.n_buffers <= 0 ? 3
                    : opt.chunk_bytes > 0 ? opt.n_buffers
                                          : std::max(opt.n_buffers, 3);
  const int nslots = static_cast<int>(std::min<int64_t>(asked, total_chunks));
  const int ns = call_streams(opt);
  const bool ring_new =
      !pinned && ensure_ring(ctx, nslots, static_cast<size_t>(std::min(per * row, out_bytes)));
  const bool exact = opt.gather_threads > 0;
  const unsigned parts = exact ? static_cast<unsigned>(opt.gather_threads) : kStagingThreads;
  ensure_workers(ctx, parts, exact);
  if (ctx.unsynced) { // a submitted upload may still read the arena this call writes
    HIPCHECK(hipStreamWaitEvent(ctx.compute, ctx.done_ev, 0));
    copy_streams_wait(ctx, ctx.done_ev);
  }
  // The source is produced on the caller's stream (0: the null stream): the
  // kernels run after it, and each copy waits on its chunk's kernel event,
  // so the copies into the caller's destination follow too.
  CallerOrder order(ctx, opt);
  order.before(ctx.compute);
  int32_t *status = ctx.status + (ctx.status_next++ % kStatusSlots);
  if (dp.family == kFamGeneric)
    clear_status(status);
  const BoundHandle::DevParams par = context_params(ctx, h, 0);
  uint8_t *result = ctx.wire;
  uint8_t *out = static_cast<uint8_t *>(dst);
  struct Pending {
    int slot;
    int64_t off, bytes;
  };
  std::vector<Pending> pending; // copies issued, not yet copied out of their slot
  size_t next = 0;
  auto consume = [&](const Pending &p) {
    TraceRange tr("relx.d2h.copy_out", p.off / std::max<int64_t>(1, per * row));
    HIPCHECK(hipEventSynchronize(ctx.slot_ev[static_cast<size_t>(p.slot)]));
    const uint8_t *from = static_cast<const uint8_t *>(ctx.slots[static_cast<size_t>(p.slot)]);
    ctx.workers->parallel_for(p.bytes, int64_t{1} << 20, [&](int64_t x, int64_t y) {
      std::memcpy(out + p.off + x, from + x, static_cast<size_t>(y - x));
    }, parts);
  };
  int64_t chunks = 0, launches = 0;
  // The kernels run back to back on the compute stream, ahead of the copies
  // (on the copy streams a kernel would queue behind the copy before it);
  // each copy waits on its chunk's kernel event.
  int ev = 0;
  hipEvent_t ke = nullptr;
  int64_t fixed[kMaxRank] = {};
  for (int64_t o = 0; o < plan.outer; ++o) {
   int64_t rem = o; // coordinates of the axes before `axis`
   for (int j = axis - 1; j >= 0; --j) {
     fixed[j] = rem % a.pext[j];
     rem /= a.pext[j];
   }
   for (int64_t u0 = 0; u0 < units; u0 += per) {
    const int64_t u1 = std::min(units, u0 + per);
    TraceRange tr("relx.d2h.submit", chunks);
    if (axis >= 0 || u0 == 0) {
      launches += launch_all(dp, prefix_launches(dp, fixed, axis, u0, u1), src, result, par.pf,
                             par.pi, status, ctx.compute);
      ke = ctx.chunk_ev[static_cast<size_t>(ev)];
      ev = (ev + 1) % kChunkEvents;
      HIPCHECK(hipEventRecord(ke, ctx.compute));
    }
    hipStream_t cs = ctx.copy_stream(chunks, ns);
    HIPCHECK(hipStreamWaitEvent(cs, ke, 0));
    const int64_t off = (o * units + u0) * row;
    const int64_t bytes = std::min((u1 - u0) * row, out_bytes - off);
    if (pinned) {
      HIPCHECK(hipMemcpyAsync(out + off, result + off, static_cast<size_t>(bytes),
                              hipMemcpyDeviceToHost, cs));
    } else {
      const int slot = static_cast<int>(chunks % nslots);
      if (pending.size() - next >= static_cast<size_t>(nslots)) // the slot's last chunk
        consume(pending[next++]);
      HIPCHECK(hipMemcpyAsync(ctx.slots[static_cast<size_t>(slot)], result + off,
                              static_cast<size_t>(bytes), hipMemcpyDeviceToHost, cs));
      HIPCHECK(hipEventRecord(ctx.slot_ev[static_cast<size_t>(slot)], cs));
      pending.push_back({slot, off, bytes});
    }
    ++chunks;
   }
  }
  while (next < pending.size())
    consume(pending[next++]);
  join_copy_streams(ctx, ctx.copies[0], std::min<int64_t>(chunks, ns));
  HIPCHECK(hipEventRecord(ctx.done_ev, ctx.copies[0]));
  // blocking: the caller's stream needs no wait for work that has completed
  HIPCHECK(hipEventSynchronize(ctx.done_ev));
  ctx.unsynced = false;
  std::fill(ctx.slot_pending.begin(), ctx.slot_pending.end(), false);
  trim_retained(ctx);
  if (dp.family == kFamGeneric) {
    if (read_status(status))
      throw Error("channel_out_of_range", "a stage selected a channel outside its parameters");
  }
  if (report) {
    relx_report &r = *report;
    std::memset(&r, 0, sizeof(r));
    std::snprintf(r.implementation, sizeof(r.implementation), "hip_relayout_d2h");
    r.source_bytes = b.typed ? b.source_bytes : dp.wire_bytes;
    r.wire_bytes = out_bytes;
    r.destination_bytes = out_bytes;
    r.parameter_bytes = b.parameter_bytes;
    r.payload_bytes_transferred = out_bytes;
    r.chunks = chunks;
    r.kernel_launches = launches;
    r.wire_boundary = static_cast<int>(h.prep.stages.size());
    r.direct_dma = pinned ? 1 : 0;
    r.host_chunk_bytes = std::min(per * row, out_bytes);
    r.host_buffers = pinned ? 0 : nslots;
    r.staging_bytes = pinned ? 0 : static_cast<int64_t>(ctx.slots.size() * ctx.slot_bytes);
    r.staging_slots = pinned ? 0 : static_cast<int64_t>(ctx.slots.size());
    r.staging_reused = !pinned && !ring_new ? 1 : 0;
    r.copy_streams = static_cast<int>(std::min<int64_t>(ns, chunks));
  }
}

// ----------------------------------------------------------- contexts

std::unique_ptr<Context> make_context(int device, int64_t max_retained) {
  auto ctx = std::make_unique<Context>();
  ctx->device = device;
  ctx->max_retained = max_retained;
  DeviceGuard guard(device);
  for (int i = 0; i < kCopyStreams; ++i) {
    HIPCHECK(hipStreamCreateWithFlags(&ctx->copies[i], hipStreamNonBlocking));
    HIPCHECK(hipEventCreateWithFlags(&ctx->join_ev[i], hipEventDisableTiming));
  }
  HIPCHECK(hipStreamCreateWithFlags(&ctx->compute, hipStreamNonBlocking));
  HIPCHECK(hipEventCreateWithFlags(&ctx->start_ev, hipEventDisableTiming));
  HIPCHECK(hipEventCreateWithFlags(&ctx->done_ev, hipEventDisableTiming));
  for (int i = 0; i < kChunkEvents; ++i) {
    hipEvent_t e;
    HIPCHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    ctx->chunk_ev.push_back(e);
  }
  // The status flags live in pinned host memory that the kernels write
  // directly: the host clears and reads a flag with plain accesses, instead
  // of a device memset and a blocking 4-byte copy per call (15 us of a small
  // call's latency).
  const size_t flags = (kStatusSlots + kDeviceChecks + 1) * sizeof(int32_t); // + the sink
  HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&ctx->status), flags, hipHostMallocDefault));
  std::memset(ctx->status, 0, flags);
  for (uint32_t i = 0; i < kDeviceChecks; ++i)
    HIPCHECK(hipEventCreateWithFlags(&ctx->check_ev[i], hipEventDisableTiming));
  // set-up of the allocation-free upload: this device's scratch address and
  // the pinned staging of its parameter tables
  ctx->stat = &static_device(device);
  HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&ctx->param_stage), kScratchParamBytes,
                         hipHostMallocDefault));
  return ctx;
}

Context::~Context() {
  if (status) {
    DeviceScope scope(device);
    (void)hipHostFree(status);
  }
}

// Drain every stream. False when completion cannot be proven.
bool drain(Context &ctx) {
  DeviceGuard guard(ctx.device);
  bool ok = hipStreamSynchronize(ctx.compute) == hipSuccess;
  for (hipStream_t c : ctx.copies)
    ok = hipStreamSynchronize(c) == hipSuccess && ok;
  // device-resident launches on callers' streams still write their flags
  for (uint32_t i = 0; i < kDeviceChecks; ++i)
    if (ctx.check_pending[i]) {
      const bool done = hipEventSynchronize(ctx.check_ev[i]) == hipSuccess;
      ok = done && ok;
      if (done) {
        ctx.check_pending[i] = false;
        if (read_status(ctx.status + kStatusSlots + i))
          ctx.channel_error = true;
      }
    }
  return ok;
}

void destroy_context(Context &ctx) {
  DeviceGuard guard(ctx.device);
  for (void *s : ctx.slots)
    (void)hipHostFree(s);
  for (hipEvent_t e : ctx.slot_ev)
    (void)hipEventDestroy(e);
  for (hipEvent_t e : ctx.chunk_ev)
    (void)hipEventDestroy(e);
  if (ctx.start_ev)
    (void)hipEventDestroy(ctx.start_ev);
  if (ctx.done_ev)
    (void)hipEventDestroy(ctx.done_ev);
  for (hipEvent_t e : ctx.join_ev)
    if (e)
      (void)hipEventDestroy(e);
  for (hipEvent_t &e : ctx.check_ev)
    if (e) {
      (void)hipEventDestroy(e);
      e = nullptr;
    }
  for (hipEvent_t e : ctx.time_ev)
    (void)hipEventDestroy(e);
  ctx.time_ev.clear();
  if (ctx.param_stage)
    (void)hipHostFree(ctx.param_stage);
  ctx.param_stage = nullptr;
  for (auto &kv : ctx.param_cache)
    (void)hipFree(kv.second.pf);
  ctx.param_cache.clear();
  ctx.param_cache_bytes = 0;
  if (ctx.wire)
    (void)hipFree(ctx.wire);
  ctx.wire = nullptr;
  ctx.wire_cap = 0;
  for (hipStream_t c : ctx.copies)
    if (c)
      (void)hipStreamDestroy(c);
  if (ctx.compute)
    (void)hipStreamDestroy(ctx.compute);
  ctx.slots.clear();
  ctx.workers.reset();
}

uint32_t source_width(const Bound &b) {
  return b.typed ? b.source_type.width() : b.layout.element_size;
}

int64_t default_chunk_bytes(int64_t total, bool h2d, bool direct) {
  constexpr int64_t M = int64_t{1} << 20;
  auto clamp = [](int64_t v, int64_t lo, int64_t hi) { return std::min(hi, std::max(lo, v)); };
  if (h2d)
    return direct ? clamp(total / 2, 32 * M, 64 * M) : clamp(total / 4, 2 * M, 8 * M);
  return direct ? clamp(total / 4, 16 * M, 32 * M) : clamp(total / 8, 4 * M, 8 * M);
}

ChunkPlan chunk_plan(const DeviceProgram &dp, uint32_t src_width, int64_t chunk_bytes, bool direct) {
  const int64_t want_chunk =
      chunk_bytes > 0 ? chunk_bytes : default_chunk_bytes(dp.wire_bytes, true, direct);
  ChunkPlan p{};
  if (dp.chunk_axis >= 0) {
    p.units = dp.base.vext[dp.chunk_axis];
    p.unit_wire = dp.chunk_stride * dp.base.win;
    p.unit_src = dp.chunk_stride * src_width;
    int64_t per = std::max<int64_t>(1, want_chunk / std::max<int64_t>(1, p.unit_wire));
    per = std::max<int64_t>(dp.chunk_align, per / dp.chunk_align * dp.chunk_align);
    p.per_chunk = std::min(per, p.units);
  } else {
    p.units = 1;
    p.per_chunk = 1;
    p.unit_wire = dp.wire_bytes;
    p.unit_src = dp.wire_elems * src_width;
  }
  return p;
}

KernelBatches kernel_batches(const ChunkPlan &p) {
  const int64_t chunks = (p.units + p.per_chunk - 1) / p.per_chunk;
  int64_t n = kKernelBatchBytes / std::max<int64_t>(1, p.per_chunk * p.unit_wire);
  n = std::max<int64_t>(1, std::min(n, chunks / 4));
  return {p.units, n * p.per_chunk, n > 1 ? (chunks - 1) * p.per_chunk : p.units};
}

int64_t verify_launches(BoundHandle &h, uint32_t k, int64_t chunk_bytes) {
  const DeviceProgram &dp = h.program(k);
  int64_t n = 0;
  bool whole = false;
  // The boxes of one schedule partition the padded destination: their
  // elements add up to it exactly.
  int64_t total = 1;
  for (int i = 0; i < dp.base.rank; ++i)
    total *= dp.base.pext[i];
  int64_t covered = 0;
  // A kernel batch reads only the wire of its own chunks, which have landed
  // when it starts: the other copy stream may still be writing the next.
  int64_t lo = 0, hi = -1;
  auto check = [&](const KArgs &a) {
    verify_launch(dp, a, lo, hi);
    int64_t e = 1;
    for (int i = 0; i < a.rank; ++i)
      e *= a.box_ext[i];
    covered += e;
    ++n;
  };
  auto schedule_done = [&] {
    if (covered != total)
      throw Error("internal_launch_check", "launch boxes cover " + std::to_string(covered) +
                                               " of " + std::to_string(total) +
                                               " destination elements");
    covered = 0;
  };
  for (int direct = 0; direct < (chunk_bytes > 0 ? 1 : 2); ++direct) {
    const ChunkPlan p = chunk_plan(dp, source_width(*h.bound), chunk_bytes, direct != 0);
    const KernelBatches kb = kernel_batches(p);
    for (int64_t v0 = 0; v0 < p.units; v0 = kb.end(v0)) {
      const int64_t v1 = kb.end(v0);
      if (v0 % p.per_chunk || (v1 % p.per_chunk && v1 != p.units))
        throw Error("internal_launch_check", "a kernel batch does not end on a chunk boundary");
      lo = dp.chunk_axis >= 0 ? v0 * dp.chunk_stride : 0;
      hi = dp.chunk_axis >= 0 ? v1 * dp.chunk_stride : -1;
      for (const KArgs &a : box_launches(dp, v0, v1, v0 == 0, v1 == p.units))
        check(a);
    }
    lo = 0;
    hi = -1;
    schedule_done();
    whole = whole || (dp.chunk_axis >= 0 && p.units > p.per_chunk);
  }
  if (whole) {
    for (const KArgs &a : box_launches(dp, 0, 0, true, true)) // the device-resident launch
      check(a);
    schedule_done();
  }
  if (h.bound->indexed) {
    // The device gather, at the natural alignment and one element off it
    // (addresses only: nothing is dereferenced).
    const Bound &b = *h.bound;
    const uint32_t sw = b.source_type.width(), rw = b.result_type.width();
    uint8_t *const base = reinterpret_cast<uint8_t *>(uintptr_t{1} << 20);
    const void *idx = base;
    for (int shift = 0; shift < 2; ++shift) {
      const uint8_t *table = base + (uintptr_t{1} << 44) + shift * sw;
      uint8_t *dst = base + (uintptr_t{1} << 45) + shift * rw;
      const GatherPlan g = gather_plan(b, table, dst);
      const std::vector<GatherArgs> ls = gather_launches(b, g, table, dst, idx);
      verify_gather(b, g, ls, table, static_cast<size_t>(b.table_bytes), dst,
                    static_cast<size_t>(b.destination_bytes), idx);
      n += static_cast<int64_t>(ls.size());
    }
    return n;
  }
  // the device-to-host schedules (axis < 0: one whole launch)
  for (int pinned = 0; k == 0 && pinned < (chunk_bytes > 0 ? 1 : 2); ++pinned) {
    const D2hPlan d = d2h_plan(dp, chunk_bytes, pinned != 0);
    int64_t fixed[kMaxRank] = {};
    for (int64_t o = 0; o < d.outer; ++o) {
      int64_t rem = o;
      for (int j = d.axis - 1; j >= 0; --j) {
        fixed[j] = rem % dp.base.pext[j];
        rem /= dp.base.pext[j];
      }
      for (int64_t u0 = 0; u0 < d.units; u0 += d.per)
        for (const KArgs &a : prefix_launches(dp, fixed, d.axis, u0, std::min(d.units, u0 + d.per))) {
          verify_launch(dp, a);
          ++n;
        }
    }
  }
  return n;
}

// Reads device-check slot i once its launch has completed; a set flag makes
// the context's channel error sticky until synchronize reports it.
void resolve_check(Context &ctx, uint32_t i) {
  if (!ctx.check_pending[i])
    return;
  HIPCHECK(hipEventSynchronize(ctx.check_ev[i]));
  ctx.check_pending[i] = false;
  if (read_status(ctx.status + kStatusSlots + i))
    ctx.channel_error = true;
}

// Waits for every device-resident launch that reports a status; throws
// channel_out_of_range (once) when one of them set its flag.
void resolve_checks(Context &ctx) {
  for (uint32_t i = 0; i < kDeviceChecks; ++i)
    resolve_check(ctx, i);
  if (ctx.channel_error) {
    ctx.channel_error = false;
    throw Error("channel_out_of_range",
                "a device-resident launch selected a stage channel outside its parameters");
  }
}

// The program's launches on `stream` as given: 0 is the legacy null stream,
// as for the reference's kernel wrappers (void *stream = nullptr).
void relayout_device(Context &ctx, BoundHandle &h, uint32_t k, const void *wire, void *dst,
                     hipStream_t stream) {
  DeviceGuard guard(ctx.device);
  const DeviceProgram &dp = h.program(k);
  const BoundHandle::DevParams par = context_params(ctx, h, k);
  if (dp.family != kFamGeneric) {
    // Fast families have their channels proven in range when the program is
    // built; their edge boxes (element-wise) get the sink flag, never read.
    launch_program(dp, 0, 0, true, true, wire, dst, par.pf, par.pi,
                   ctx.status + kStatusSlots + kDeviceChecks, stream);
    return;
  }
  const uint32_t i = ctx.check_next++ % kDeviceChecks;
  resolve_check(ctx, i); // its previous launch, kDeviceChecks calls ago
  int32_t *status = ctx.status + kStatusSlots + i;
  clear_status(status);
  launch_program(dp, 0, 0, true, true, wire, dst, par.pf, par.pi, status, stream);
  HIPCHECK(hipEventRecord(ctx.check_ev[i], stream));
  ctx.check_pending[i] = true;
}

double measure_copy(int device, size_t bytes, int iters, int rounds, bool d2h);

double measure_h2d(int device, size_t bytes, int iters, int rounds) {
  return measure_copy(device, bytes, iters, rounds, false);
}

double measure_copy(int device, size_t bytes, int iters, int rounds, bool d2h) {
  DeviceGuard guard(device);
  void *h = nullptr, *d = nullptr;
  hipStream_t s;
  hipEvent_t e0, e1;
  HIPCHECK(hipHostMalloc(&h, bytes, hipHostMallocDefault));
  HIPCHECK(hipMalloc(&d, bytes));
  std::memset(h, 1, bytes);
  HIPCHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  HIPCHECK(hipEventCreate(&e0));
  HIPCHECK(hipEventCreate(&e1));
  auto copy = [&] {
    return d2h ? hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, s)
               : hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s);
  };
  for (int i = 0; i < 3; ++i)
    HIPCHECK(copy());
  HIPCHECK(hipStreamSynchronize(s));
  double best = 0.0;
  for (int r = 0; r < rounds; ++r) {
    HIPCHECK(hipEventRecord(e0, s));
    for (int i = 0; i < iters; ++i)
      HIPCHECK(copy());
    HIPCHECK(hipEventRecord(e1, s));
    HIPCHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
    best = std::max(best, static_cast<double>(bytes) * iters / (ms * 1e-3) / 1e9);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipStreamDestroy(s);
  (void)hipFree(d);
  (void)hipHostFree(h);
  return best;
}

hipError_t copy16_launch(const void *src, void *dst, uint32_t n16, int items, hipStream_t s);

double measure_device_copy(int device, size_t bytes, int iters, int rounds) {
  DeviceGuard guard(device);
  const size_t n16 = bytes / 16;
  if (n16 == 0 || n16 >= (size_t{1} << 31))
    throw Error("invalid_argument", "copy size must be 16 B to 32 GiB");
  bytes = n16 * 16;
  // Rotate buffer pairs spanning at least 2 GiB, eight times the 256 MB
  // Infinity Cache, and make each timed round at least one pass over them, so
  // every copy reads and writes HBM (a destination still held in the cache
  // from an earlier pass would absorb the rewrite).
  const size_t sets = std::max<size_t>(2, ((size_t{2} << 30) + 2 * bytes - 1) / (2 * bytes));
  iters = std::max(iters, static_cast<int>(sets));
  std::vector<void *> src(sets, nullptr), dst(sets, nullptr);
  hipStream_t s = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  double best = 0.0;
  auto release = [&] {
    for (void *p : src)
      (void)hipFree(p);
    for (void *p : dst)
      (void)hipFree(p);
    if (e0)
      (void)hipEventDestroy(e0);
    if (e1)
      (void)hipEventDestroy(e1);
    if (s)
      (void)hipStreamDestroy(s);
  };
  try {
    for (size_t i = 0; i < sets; ++i) {
      HIPCHECK(hipMalloc(&src[i], bytes));
      HIPCHECK(hipMalloc(&dst[i], bytes));
      HIPCHECK(hipMemset(src[i], 1, bytes));
    }
    HIPCHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    HIPCHECK(hipEventCreate(&e0));
    HIPCHECK(hipEventCreate(&e1));
    // both forms of the copy (one and two vectors per lane), the faster one
    // counts: one is faster from about 128 MB up, two below
    for (int items = 1; items <= 2; ++items) {
      for (size_t i = 0; i < 2 * sets; ++i)
        HIPCHECK(copy16_launch(src[i % sets], dst[i % sets], static_cast<uint32_t>(n16), items, s));
      HIPCHECK(hipStreamSynchronize(s));
      for (int r = 0; r < rounds; ++r) {
        HIPCHECK(hipEventRecord(e0, s));
        for (int i = 0; i < iters; ++i)
          HIPCHECK(copy16_launch(src[static_cast<size_t>(i) % sets],
                                 dst[static_cast<size_t>(i) % sets], static_cast<uint32_t>(n16),
                                 items, s));
        HIPCHECK(hipEventRecord(e1, s));
        HIPCHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
        best = std::max(best, 2.0 * static_cast<double>(bytes) * iters / (ms * 1e-3) / 1e9);
      }
    }
  } catch (...) {
    release();
    throw;
  }
  release();
  return best;
}

} // namespace relx
