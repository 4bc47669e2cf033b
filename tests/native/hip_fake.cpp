// hip_fake.cpp - a CPU stand-in for the HIP runtime calls librelx's host
// sources make, with an ordering checker and fault knobs (see hip_fake.h).
// Test infrastructure: linked only into tests/native/pipeline_driver.
//
// Kernels: every relayout launch is run with the element-wise kernel's
// semantics (sym_amd/csrc/kernels.h, k_generic), which every family's
// launch arguments also describe (the library itself falls back to it for
// unaligned buffers); value stages are not run (counted as unemulated), so
// result bytes are checked only for programs without device stages. Row
// gathers run for plain copies; copy16 copies.
#include "hip_fake.h"

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "program.h"
#include "runtime.h"

namespace {

using VClock = std::vector<uint64_t>;

void vjoin(VClock &a, const VClock &b) {
  if (a.size() < b.size())
    a.resize(b.size(), 0);
  for (size_t i = 0; i < b.size(); ++i)
    a[i] = std::max(a[i], b[i]);
}

uint64_t vget(const VClock &c, int i) {
  return i >= 0 && static_cast<size_t>(i) < c.size() ? c[static_cast<size_t>(i)] : 0;
}

void vtick(VClock &c, int i) {
  if (c.size() <= static_cast<size_t>(i))
    c.resize(static_cast<size_t>(i) + 1, 0);
  ++c[static_cast<size_t>(i)];
}

std::mutex g_mu; // guards everything below
std::condition_variable g_cv;
int g_next_agent = 0;

// One hipEventRecord: done when its stream reaches it.
struct Record {
  bool done = false;
  std::chrono::steady_clock::time_point ts;
  VClock vc;
};

enum class OpKind { Data, Marker, Wait };

struct Op {
  OpKind kind = OpKind::Data;
  std::function<void()> run;
  int delay_us = 0;
  bool fault = false;
  int device = 0;
  std::shared_ptr<Record> rec;
};

enum class Mem { Device, Pinned, UserHost };

struct Alloc {
  size_t bytes;
  Mem kind;
  int device;
  bool user; // pinned memory the caller owns (not the library's staging)
};

std::map<uintptr_t, Alloc> g_allocs;

// The destination elements of a relayout launch: a box of padded
// coordinates mapped by the program's strides. Two boxes of one program
// (same base, strides and element size) share no element unless they
// overlap on every axis, though their byte spans may interleave.
struct BoxShape {
  bool set = false;
  uintptr_t base = 0;
  int rank = 0, width = 0;
  int64_t lo[relx::kMaxRank] = {}, ext[relx::kMaxRank] = {}, ds[relx::kMaxRank] = {};
};

bool same_program(const BoxShape &a, const BoxShape &b) {
  if (!a.set || !b.set || a.base != b.base || a.rank != b.rank || a.width != b.width)
    return false;
  for (int k = 0; k < a.rank; ++k)
    if (a.ds[k] != b.ds[k])
      return false;
  return true;
}

bool boxes_disjoint(const BoxShape &a, const BoxShape &b) {
  for (int k = 0; k < a.rank; ++k)
    if (a.lo[k] + a.ext[k] <= b.lo[k] || b.lo[k] + b.ext[k] <= a.lo[k])
      return true;
  return false;
}

struct Access {
  uintptr_t lo, hi;
  int agent;
  uint64_t seq;
  bool write;
  std::string what;
  BoxShape box;
};
std::vector<Access> g_acc;
std::vector<std::string> g_violations;
std::vector<VClock> g_tokens; // host hand-off snapshots

fake_knobs g_knobs{};
fake_counts g_counts{};
std::mt19937 g_rng(1);
hipError_t g_sticky[8] = {};

struct HostAgent {
  int id = -1;
  VClock vc;
};
thread_local HostAgent t_host;
thread_local uint64_t t_call = 0; // library calls this thread has begun
// Per library staging allocation: who last staged it (host agent, call,
// destination of the kernels that read it).
struct Staged {
  int agent;
  uint64_t call;
  const void *dst;
  bool operator==(const Staged &o) const {
    return agent == o.agent && call == o.call && dst == o.dst;
  }
};
std::map<uintptr_t, Staged> g_staged;
thread_local int t_device = 0;
thread_local hipError_t t_last = hipSuccess;

// Under g_mu: the calling thread's agent, advanced by one action.
HostAgent &host_tick() {
  if (t_host.id < 0)
    t_host.id = g_next_agent++;
  vtick(t_host.vc, t_host.id);
  return t_host;
}

void violation(const std::string &s) {
  if (g_violations.size() < 200)
    g_violations.push_back(s);
}

const Alloc *find_alloc(uintptr_t p, uintptr_t *base = nullptr) {
  auto it = g_allocs.upper_bound(p);
  if (it == g_allocs.begin())
    return nullptr;
  --it;
  if (p >= it->first + it->second.bytes)
    return nullptr;
  if (base)
    *base = it->first;
  return &it->second;
}

std::string describe(uintptr_t lo, uintptr_t hi) {
  uintptr_t base = 0;
  const Alloc *a = find_alloc(lo, &base);
  char buf[160];
  const char *kind = !a ? "untracked" : a->kind == Mem::Device ? "device" : a->kind == Mem::Pinned ? "pinned" : "host";
  std::snprintf(buf, sizeof(buf), "%s[%#lx +%lu, %lu bytes)", kind, static_cast<unsigned long>(base),
                static_cast<unsigned long>(lo - base), static_cast<unsigned long>(hi - lo));
  return buf;
}

// Under g_mu: an access by `agent` at step `seq` whose clock is `vc`, checked
// against the earlier conflicting accesses to the same bytes, then recorded.
// Only tracked memory is checked.
void access(uintptr_t lo, uintptr_t hi, bool write, const VClock &vc, int agent, uint64_t seq,
            const std::string &what, const BoxShape &box = BoxShape()) {
  if (hi <= lo || !find_alloc(lo))
    return;
  for (const Access &a : g_acc) {
    if (a.hi <= lo || hi <= a.lo || (!a.write && !write) || a.agent == agent)
      continue;
    if (same_program(a.box, box) && boxes_disjoint(a.box, box))
      continue;
    if (vget(vc, a.agent) < a.seq)
      violation(what + " " + (write ? "writes " : "reads ") + describe(lo, hi) +
                " unordered with an earlier " + (a.write ? "write" : "read") + " by " + a.what);
  }
  g_acc.push_back(Access{lo, hi, agent, seq, write, what, box});
}

// Under g_mu: a device access must lie inside one tracked allocation of the
// given kind (device memory for kernels and device ends of copies).
bool inside(uintptr_t lo, uintptr_t hi, Mem kind, const char *what) {
  if (hi <= lo)
    return true;
  uintptr_t base = 0;
  const Alloc *a = find_alloc(lo, &base);
  if (!a || a->kind != kind || hi > base + a->bytes) {
    violation(std::string(what) + ": " + describe(lo, hi) + " is outside a " +
              (kind == Mem::Device ? "device" : "page-locked") + " allocation");
    return false;
  }
  return true;
}

// A kernel reads device memory, or the library's own page-locked staging (a
// zero-copy chunk); never page-locked memory of the caller.
bool kernel_readable(uintptr_t lo, uintptr_t hi, const char *what) {
  if (hi <= lo)
    return true;
  uintptr_t base = 0;
  const Alloc *a = find_alloc(lo, &base);
  if (a && a->kind == Mem::Pinned && !a->user && hi <= base + a->bytes)
    return true;
  return inside(lo, hi, Mem::Device, what);
}

int pick_delay(int d) {
  if (d <= 0)
    return 0;
  if (!g_knobs.jitter)
    return d;
  return static_cast<int>(g_rng() % static_cast<uint32_t>(d + 1));
}

} // namespace

struct ihipStream_t {
  int agent = 0;
  int device = 0;
  bool null_stream = false;
  std::deque<Op> q;
  bool stop = false;
  VClock vc;
  std::thread worker;
};

struct ihipEvent_t {
  bool timing = true;
  std::shared_ptr<Record> last;
};

namespace {

std::vector<ihipStream_t *> g_streams; // every live stream (for shutdown)
ihipStream_t *g_null[8] = {};

void worker_loop(ihipStream_t *s) {
  std::unique_lock<std::mutex> lk(g_mu);
  for (;;) {
    g_cv.wait(lk, [&] { return s->stop || !s->q.empty(); });
    if (s->q.empty())
      return;
    Op &op = s->q.front(); // deque references survive push_back
    switch (op.kind) {
    case OpKind::Wait: {
      std::shared_ptr<Record> r = op.rec;
      g_cv.wait(lk, [&] { return r->done; });
      break;
    }
    case OpKind::Marker:
      op.rec->done = true;
      op.rec->ts = std::chrono::steady_clock::now();
      break;
    case OpKind::Data: {
      const bool skip = g_sticky[op.device] != hipSuccess;
      std::function<void()> run = std::move(op.run);
      const int delay = op.delay_us;
      const bool fault = op.fault;
      lk.unlock();
      if (delay > 0)
        std::this_thread::sleep_for(std::chrono::microseconds(delay));
      if (!skip && !fault && run)
        run();
      lk.lock();
      if (fault)
        g_sticky[op.device] = hipErrorIllegalAddress;
      break;
    }
    }
    s->q.pop_front();
    g_cv.notify_all();
  }
}

ihipStream_t *new_stream(int device, bool null_stream) {
  auto *s = new ihipStream_t;
  s->agent = g_next_agent++;
  s->device = device;
  s->null_stream = null_stream;
  s->worker = std::thread(worker_loop, s);
  g_streams.push_back(s);
  return s;
}

// Under g_mu.
ihipStream_t *resolve(hipStream_t s) {
  if (s)
    return s;
  const int d = t_device;
  if (!g_null[d])
    g_null[d] = new_stream(d, true);
  return g_null[d];
}

// Under g_mu: the stream's clock after this host action, and the op's step.
uint64_t stream_step(ihipStream_t *s) {
  HostAgent &h = host_tick();
  vjoin(s->vc, h.vc);
  vtick(s->vc, s->agent);
  return s->vc[static_cast<size_t>(s->agent)];
}

void push(ihipStream_t *s, Op op) {
  s->q.push_back(std::move(op));
  g_cv.notify_all();
}

hipError_t set_last(hipError_t e) {
  if (e != hipSuccess)
    t_last = e;
  return e;
}

bool nth(int64_t count, int at) { return at > 0 && count == at; }

// Under g_mu: enqueue a copy with its accesses. `host_writes` marks a source
// in the library's own page-locked staging, which the host has just filled.
hipError_t enqueue_copy(void *dst, const void *src, size_t n, hipMemcpyKind kind, hipStream_t hs,
                        const char *what) {
  ihipStream_t *s = resolve(hs);
  if (g_sticky[s->device] != hipSuccess)
    return g_sticky[s->device];
  const int64_t nc = ++g_counts.copies;
  if (nth(nc, g_knobs.fail_copy_at))
    return hipErrorInvalidValue;
  const uintptr_t d = reinterpret_cast<uintptr_t>(dst), sp = reinterpret_cast<uintptr_t>(src);
  bool ok = true;
  if (kind == hipMemcpyHostToDevice || kind == hipMemcpyDeviceToDevice)
    ok = inside(d, d + n, Mem::Device, what) && ok;
  if (kind == hipMemcpyDeviceToHost || kind == hipMemcpyDeviceToDevice)
    ok = inside(sp, sp + n, Mem::Device, what) && ok;
  if (!ok)
    return hipErrorInvalidValue;
  if (kind == hipMemcpyHostToDevice) {
    const Alloc *a = find_alloc(sp);
    if (a && a->kind == Mem::Pinned && !a->user) {
      HostAgent &h = host_tick();
      access(sp, sp + n, true, h.vc, h.id, h.vc[static_cast<size_t>(h.id)], "host staging write");
    }
  }
  const uint64_t seq = stream_step(s);
  char tag[96];
  std::snprintf(tag, sizeof(tag), "%s (stream %d, step %lu)", what, s->agent,
                static_cast<unsigned long>(seq));
  access(sp, sp + n, false, s->vc, s->agent, seq, tag);
  access(d, d + n, true, s->vc, s->agent, seq, tag);
  Op op;
  op.device = s->device;
  op.delay_us = pick_delay(g_knobs.delay_copy_us);
  op.fault = nth(nc, g_knobs.fail_copy_async_at);
  op.run = [dst, src, n] { std::memcpy(dst, src, n); };
  push(s, std::move(op));
  return hipSuccess;
}

// Under g_mu: wait for a stream to run dry.
hipError_t wait_stream(std::unique_lock<std::mutex> &lk, ihipStream_t *s) {
  const int64_t n = ++g_counts.syncs;
  if (g_knobs.sync_unknown || nth(n, g_knobs.fail_sync_at))
    return hipErrorUnknown;
  g_cv.wait(lk, [&] { return s->q.empty(); });
  HostAgent &h = host_tick();
  vjoin(h.vc, s->vc);
  return g_sticky[s->device];
}

void *raw_alloc(size_t bytes) {
  const size_t n = (std::max<size_t>(bytes, 1) + 255) / 256 * 256;
  return std::aligned_alloc(256, n);
}

// Under g_mu: release an allocation the host frees; every access to it
// must be ordered before the host.
hipError_t release(void *p, Mem kind, const char *what) {
  if (!p)
    return hipSuccess;
  auto it = g_allocs.find(reinterpret_cast<uintptr_t>(p));
  if (it == g_allocs.end() || it->second.kind != kind) {
    violation(std::string(what) + " of a pointer that is not an allocation of that kind");
    return hipErrorInvalidValue;
  }
  const uintptr_t lo = it->first, hi = lo + it->second.bytes;
  HostAgent &h = host_tick();
  const size_t before = g_violations.size();
  access(lo, hi, true, h.vc, h.id, h.vc[static_cast<size_t>(h.id)], what);
  const bool in_use = g_violations.size() != before;
  g_acc.erase(std::remove_if(g_acc.begin(), g_acc.end(),
                             [&](const Access &a) { return a.lo < hi && lo < a.hi; }),
              g_acc.end());
  g_staged.erase(lo);
  g_allocs.erase(it);
  if (!in_use) // memory a device operation may still touch is kept
    std::free(p);
  return hipSuccess;
}

// Element loads and stores of 1, 2, 4 or 8 bytes (little endian).
uint64_t load_el(const uint8_t *p, int w) {
  uint64_t x = 0;
  std::memcpy(&x, p, static_cast<size_t>(w));
  return x;
}

void store_el(uint8_t *p, uint64_t x, int w) { std::memcpy(p, &x, static_cast<size_t>(w)); }

// The element-wise kernel's loop over a launch box (no value stages).
void run_box(const relx::KArgs &a) {
  int64_t work = 1;
  for (int k = 0; k < a.rank; ++k)
    work *= a.box_ext[k];
  for (int64_t i = 0; i < work; ++i) {
    int64_t rem = i, dof = 0, sof = 0;
    bool pad = false;
    for (int k = a.rank - 1; k >= 0; --k) {
      const int64_t e = a.box_ext[k];
      const int64_t p = rem % e + a.box_lo[k];
      rem /= e;
      dof += p * a.ds[k];
      const int64_t v = p - a.lo[k];
      if (v < 0 || v >= a.vext[k])
        pad = true;
      else
        sof += v * a.ss[k];
    }
    const uint64_t x = pad ? a.fill64 : load_el(a.src + sof * a.win, a.win);
    store_el(a.dst + dof * a.wout, x, a.wout);
  }
}

// Byte spans a box reads and writes: [min, max] offsets per axis.
void box_spans(const relx::KArgs &a, uintptr_t &slo, uintptr_t &shi, uintptr_t &dlo, uintptr_t &dhi) {
  int64_t smin = 0, smax = 0, dmin = 0, dmax = 0;
  bool valid = true;
  for (int k = 0; k < a.rank; ++k) {
    const int64_t p0 = a.box_lo[k], p1 = a.box_lo[k] + a.box_ext[k] - 1;
    dmin += std::min(p0 * a.ds[k], p1 * a.ds[k]);
    dmax += std::max(p0 * a.ds[k], p1 * a.ds[k]);
    const int64_t v0 = std::max<int64_t>(p0 - a.lo[k], 0), v1 = std::min(p1 - a.lo[k], a.vext[k] - 1);
    if (v0 > v1) {
      valid = false;
    } else {
      smin += std::min(v0 * a.ss[k], v1 * a.ss[k]);
      smax += std::max(v0 * a.ss[k], v1 * a.ss[k]);
    }
  }
  const uintptr_t s = reinterpret_cast<uintptr_t>(a.src), d = reinterpret_cast<uintptr_t>(a.dst);
  slo = shi = s;
  if (valid) {
    slo = s + static_cast<uintptr_t>(smin * a.win);
    shi = s + static_cast<uintptr_t>((smax + 1) * a.win);
  }
  dlo = d + static_cast<uintptr_t>(dmin * a.wout);
  dhi = d + static_cast<uintptr_t>((dmax + 1) * a.wout);
}

// Under g_mu: enqueue a kernel whose accesses are given.
hipError_t enqueue_kernel(hipStream_t hs, const char *what,
                          const std::vector<std::pair<uintptr_t, uintptr_t>> &reads,
                          std::pair<uintptr_t, uintptr_t> write, std::function<void()> run,
                          const BoxShape &box = BoxShape()) {
  ihipStream_t *s = resolve(hs);
  if (g_sticky[s->device] != hipSuccess)
    return g_sticky[s->device];
  const int64_t n = ++g_counts.launches;
  if (nth(n, g_knobs.fail_launch_at))
    return hipErrorLaunchFailure;
  bool ok = inside(write.first, write.second, Mem::Device, what);
  for (const auto &r : reads)
    ok = kernel_readable(r.first, r.second, what) && ok;
  if (!ok)
    return hipErrorInvalidValue;
  const uint64_t seq = stream_step(s);
  char tag[96];
  std::snprintf(tag, sizeof(tag), "%s (stream %d, step %lu)", what, s->agent,
                static_cast<unsigned long>(seq));
  for (const auto &r : reads)
    access(r.first, r.second, false, s->vc, s->agent, seq, tag);
  access(write.first, write.second, true, s->vc, s->agent, seq, tag, box);
  Op op;
  op.device = s->device;
  op.delay_us = pick_delay(g_knobs.delay_kernel_us);
  op.fault = nth(n, g_knobs.fail_kernel_async_at);
  op.run = std::move(run);
  push(s, std::move(op));
  return hipSuccess;
}

const char *error_name(hipError_t e) {
  switch (e) {
  case hipSuccess:
    return "hipSuccess";
  case hipErrorInvalidValue:
    return "hipErrorInvalidValue";
  case hipErrorOutOfMemory:
    return "hipErrorOutOfMemory";
  case hipErrorInvalidDevice:
    return "hipErrorInvalidDevice";
  case hipErrorInvalidHandle:
    return "hipErrorInvalidHandle";
  case hipErrorNotReady:
    return "hipErrorNotReady";
  case hipErrorLaunchFailure:
    return "hipErrorLaunchFailure";
  case hipErrorIllegalAddress:
    return "hipErrorIllegalAddress";
  case hipErrorUnknown:
    return "hipErrorUnknown";
  default:
    return "hipError(other)";
  }
}

} // namespace

// ------------------------------------------------------------ HIP calls

hipError_t hipGetDeviceCount(int *count) {
  std::lock_guard<std::mutex> g(g_mu);
  *count = g_knobs.device_count > 0 ? g_knobs.device_count : 1;
  return hipSuccess;
}

hipError_t hipSetDevice(int d) {
  std::lock_guard<std::mutex> g(g_mu);
  const int n = g_knobs.device_count > 0 ? g_knobs.device_count : 1;
  if (d < 0 || d >= n)
    return set_last(hipErrorInvalidDevice);
  t_device = d;
  return hipSuccess;
}

hipError_t hipGetDevice(int *d) {
  *d = t_device;
  return hipSuccess;
}

hipError_t hipGetLastError(void) {
  const hipError_t e = t_last;
  t_last = hipSuccess;
  return e;
}

const char *hipGetErrorString(hipError_t e) { return error_name(e); }

hipError_t hipMalloc(void **ptr, size_t size) {
  std::lock_guard<std::mutex> g(g_mu);
  if (nth(++g_counts.mallocs, g_knobs.fail_malloc_at))
    return set_last(hipErrorOutOfMemory);
  void *p = raw_alloc(size);
  std::memset(p, 0xCD, size); // fresh device memory holds garbage
  g_allocs[reinterpret_cast<uintptr_t>(p)] = Alloc{size, Mem::Device, t_device, false};
  ++g_counts.live_device;
  *ptr = p;
  return hipSuccess;
}

hipError_t hipFree(void *ptr) {
  std::lock_guard<std::mutex> g(g_mu);
  if (!ptr)
    return hipSuccess;
  ++g_counts.frees;
  const hipError_t e = release(ptr, Mem::Device, "hipFree");
  if (e == hipSuccess)
    --g_counts.live_device;
  return e;
}

hipError_t hipHostMalloc(void **ptr, size_t size, unsigned int) {
  std::lock_guard<std::mutex> g(g_mu);
  if (nth(++g_counts.host_mallocs, g_knobs.fail_host_malloc_at))
    return set_last(hipErrorOutOfMemory);
  void *p = raw_alloc(size);
  std::memset(p, 0xEE, size);
  g_allocs[reinterpret_cast<uintptr_t>(p)] = Alloc{size, Mem::Pinned, t_device, false};
  ++g_counts.live_pinned;
  *ptr = p;
  return hipSuccess;
}

hipError_t hipHostFree(void *ptr) {
  std::lock_guard<std::mutex> g(g_mu);
  if (!ptr)
    return hipSuccess;
  ++g_counts.host_frees;
  const hipError_t e = release(ptr, Mem::Pinned, "hipHostFree");
  if (e == hipSuccess)
    --g_counts.live_pinned;
  return e;
}

hipError_t hipPointerGetAttributes(hipPointerAttribute_t *attr, const void *ptr) {
  std::lock_guard<std::mutex> g(g_mu);
  const Alloc *a = find_alloc(reinterpret_cast<uintptr_t>(ptr));
  if (!a || a->kind == Mem::UserHost)
    return set_last(hipErrorInvalidValue);
  std::memset(attr, 0, sizeof(*attr));
  attr->type = a->kind == Mem::Device ? hipMemoryTypeDevice : hipMemoryTypeHost;
  attr->device = a->device;
  attr->devicePointer = const_cast<void *>(ptr);
  attr->hostPointer = a->kind == Mem::Pinned ? const_cast<void *>(ptr) : nullptr;
  return hipSuccess;
}

hipError_t hipStreamCreateWithFlags(hipStream_t *stream, unsigned int) {
  std::lock_guard<std::mutex> g(g_mu);
  *stream = new_stream(t_device, false);
  return hipSuccess;
}

hipError_t hipStreamDestroy(hipStream_t stream) {
  std::unique_lock<std::mutex> lk(g_mu);
  if (!stream)
    return set_last(hipErrorInvalidHandle);
  g_cv.wait(lk, [&] { return stream->q.empty(); });
  stream->stop = true;
  g_cv.notify_all();
  g_streams.erase(std::remove(g_streams.begin(), g_streams.end(), stream), g_streams.end());
  lk.unlock();
  stream->worker.join();
  delete stream;
  return hipSuccess;
}

hipError_t hipStreamSynchronize(hipStream_t stream) {
  std::unique_lock<std::mutex> lk(g_mu);
  return set_last(wait_stream(lk, resolve(stream)));
}

// Complete when every operation enqueued on the stream has run; the host is
// then ordered after all of them, as after a synchronize.
hipError_t hipStreamQuery(hipStream_t stream) {
  std::lock_guard<std::mutex> g(g_mu);
  ihipStream_t *s = resolve(stream);
  if (g_sticky[s->device] != hipSuccess)
    return set_last(g_sticky[s->device]);
  if (!s->q.empty())
    return hipErrorNotReady;
  HostAgent &h = host_tick();
  vjoin(h.vc, s->vc);
  return hipSuccess;
}

hipError_t hipStreamWaitEvent(hipStream_t stream, hipEvent_t event, unsigned int) {
  std::lock_guard<std::mutex> g(g_mu);
  ihipStream_t *s = resolve(stream);
  if (g_sticky[s->device] != hipSuccess)
    return set_last(g_sticky[s->device]);
  if (nth(++g_counts.waits, g_knobs.fail_wait_at))
    return set_last(hipErrorInvalidHandle);
  HostAgent &h = host_tick();
  vjoin(s->vc, h.vc);
  if (!event->last)
    return hipSuccess; // never recorded: nothing to wait for
  vjoin(s->vc, event->last->vc);
  Op op;
  op.kind = OpKind::Wait;
  op.device = s->device;
  op.rec = event->last;
  push(s, std::move(op));
  return hipSuccess;
}

hipError_t hipEventCreate(hipEvent_t *event) {
  *event = new ihipEvent_t;
  return hipSuccess;
}

hipError_t hipEventCreateWithFlags(hipEvent_t *event, unsigned flags) {
  *event = new ihipEvent_t;
  (*event)->timing = (flags & hipEventDisableTiming) == 0;
  return hipSuccess;
}

hipError_t hipEventDestroy(hipEvent_t event) {
  delete event; // pending operations hold their records, not the event
  return hipSuccess;
}

hipError_t hipEventRecord(hipEvent_t event, hipStream_t stream) {
  std::lock_guard<std::mutex> g(g_mu);
  ihipStream_t *s = resolve(stream);
  if (g_sticky[s->device] != hipSuccess)
    return set_last(g_sticky[s->device]);
  if (nth(++g_counts.records, g_knobs.fail_record_at))
    return set_last(hipErrorInvalidHandle);
  stream_step(s);
  auto rec = std::make_shared<Record>();
  rec->vc = s->vc;
  event->last = rec;
  Op op;
  op.kind = OpKind::Marker;
  op.device = s->device;
  op.rec = rec;
  push(s, std::move(op));
  return hipSuccess;
}

hipError_t hipEventSynchronize(hipEvent_t event) {
  std::unique_lock<std::mutex> lk(g_mu);
  const int64_t n = ++g_counts.syncs;
  if (g_knobs.sync_unknown || nth(n, g_knobs.fail_sync_at))
    return set_last(hipErrorUnknown);
  std::shared_ptr<Record> r = event->last;
  if (!r)
    return hipSuccess;
  g_cv.wait(lk, [&] { return r->done; });
  HostAgent &h = host_tick();
  vjoin(h.vc, r->vc);
  return set_last(g_sticky[t_device]);
}

hipError_t hipEventQuery(hipEvent_t event) {
  std::lock_guard<std::mutex> g(g_mu);
  if (g_sticky[t_device] != hipSuccess)
    return set_last(g_sticky[t_device]);
  std::shared_ptr<Record> r = event->last;
  if (!r)
    return hipSuccess;
  if (!r->done)
    return hipErrorNotReady;
  HostAgent &h = host_tick();
  vjoin(h.vc, r->vc);
  return hipSuccess;
}

hipError_t hipEventElapsedTime(float *ms, hipEvent_t start, hipEvent_t stop) {
  std::lock_guard<std::mutex> g(g_mu);
  if (!start->timing || !stop->timing || !start->last || !stop->last)
    return set_last(hipErrorInvalidHandle);
  if (!start->last->done || !stop->last->done)
    return hipErrorNotReady;
  *ms = std::chrono::duration<float, std::milli>(stop->last->ts - start->last->ts).count();
  return hipSuccess;
}

hipError_t hipMemcpyAsync(void *dst, const void *src, size_t sizeBytes, hipMemcpyKind kind,
                          hipStream_t stream) {
  std::lock_guard<std::mutex> g(g_mu);
  const char *what = kind == hipMemcpyHostToDevice   ? "H2D copy"
                     : kind == hipMemcpyDeviceToHost ? "D2H copy"
                                                     : "copy";
  return set_last(enqueue_copy(dst, src, sizeBytes, kind, stream, what));
}

hipError_t hipMemcpy(void *dst, const void *src, size_t sizeBytes, hipMemcpyKind kind) {
  std::unique_lock<std::mutex> lk(g_mu);
  hipError_t e = enqueue_copy(dst, src, sizeBytes, kind, nullptr, "blocking copy");
  if (e == hipSuccess) {
    ihipStream_t *s = resolve(nullptr);
    g_cv.wait(lk, [&] { return s->q.empty(); });
    HostAgent &h = host_tick();
    vjoin(h.vc, s->vc);
    e = g_sticky[s->device];
  }
  return set_last(e);
}

hipError_t hipMemset(void *dst, int value, size_t sizeBytes) {
  std::unique_lock<std::mutex> lk(g_mu);
  const uintptr_t d = reinterpret_cast<uintptr_t>(dst);
  if (!inside(d, d + sizeBytes, Mem::Device, "hipMemset"))
    return set_last(hipErrorInvalidValue);
  ihipStream_t *s = resolve(nullptr);
  const uint64_t seq = stream_step(s);
  access(d, d + sizeBytes, true, s->vc, s->agent, seq, "hipMemset");
  Op op;
  op.device = s->device;
  op.run = [dst, value, sizeBytes] { std::memset(dst, value, sizeBytes); };
  push(s, std::move(op));
  g_cv.wait(lk, [&] { return s->q.empty(); });
  HostAgent &h = host_tick();
  vjoin(h.vc, s->vc);
  return set_last(g_sticky[s->device]);
}

// ------------------------------------------------- device entry points

namespace relx {

hipError_t launch_box(int family, const KArgs &a, int32_t *status, hipStream_t s) {
  (void)family;
  (void)status;
  if (a.work64 <= 0)
    return hipSuccess;
  uintptr_t slo, shi, dlo, dhi;
  box_spans(a, slo, shi, dlo, dhi);
  std::lock_guard<std::mutex> g(g_mu);
  const bool stages = a.chain.n > 0;
  if (stages)
    ++g_counts.unemulated;
  {
    // a kernel that reads the library's own page-locked staging (a
    // zero-copy chunk): the host has just filled it, as for a copy from it
    // (once per chunk: the chunk's later kernels read the same staging)
    uintptr_t base = 0;
    const Alloc *al = find_alloc(slo, &base);
    if (al && al->kind == Mem::Pinned && !al->user) {
      ++g_counts.zero_copy;
      HostAgent &h = host_tick();
      const Staged now{h.id, t_call, a.dst};
      auto it = g_staged.find(base);
      if (t_call == 0 || it == g_staged.end() || !(it->second == now)) {
        access(slo, shi, true, h.vc, h.id, h.vc[static_cast<size_t>(h.id)], "host staging write");
        g_staged[base] = now;
      }
    }
  }
  std::vector<std::pair<uintptr_t, uintptr_t>> reads{{slo, shi}};
  // parameter tables: from the table to the end of its allocation
  for (const void *p : {static_cast<const void *>(a.pf), static_cast<const void *>(a.pi)}) {
    uintptr_t base = 0;
    const uintptr_t q = reinterpret_cast<uintptr_t>(p);
    const Alloc *al = p ? find_alloc(q, &base) : nullptr;
    if (stages && al)
      reads.push_back({q, base + al->bytes});
  }
  BoxShape box;
  box.set = true;
  box.base = reinterpret_cast<uintptr_t>(a.dst);
  box.rank = a.rank;
  box.width = a.wout;
  for (int i = 0; i < a.rank; ++i) {
    box.lo[i] = a.box_lo[i];
    box.ext[i] = a.box_ext[i];
    box.ds[i] = a.ds[i];
  }
  const KArgs k = a;
  return set_last(enqueue_kernel(s, "relayout kernel", reads, {dlo, dhi}, [k] { run_box(k); }, box));
}

hipError_t gather_launch(const GatherArgs &a, int op, int nbi, int iw, bool nt, hipStream_t s) {
  (void)nt;
  if (a.work == 0)
    return hipSuccess;
  const int nbo = op == kGatherF32F16 ? nbi / 2 : op == kGatherF16F32 ? nbi * 2 : nbi;
  const int64_t rows = (static_cast<int64_t>(a.work) + a.row_items - 1) / a.row_items;
  const int64_t row_bytes = static_cast<int64_t>(a.row_items) * nbi;
  std::lock_guard<std::mutex> g(g_mu);
  const uintptr_t ix = reinterpret_cast<uintptr_t>(a.idx);
  if (!inside(ix, ix + static_cast<uintptr_t>(rows * iw), Mem::Device, "row gather indices"))
    return set_last(hipErrorInvalidValue);
  int64_t lo = INT64_MAX, hi = -1; // the rows read (the indices were uploaded by a blocking copy)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t v = iw == 8 ? reinterpret_cast<const int64_t *>(a.idx)[r]
                              : reinterpret_cast<const int32_t *>(a.idx)[r];
    lo = std::min(lo, v);
    hi = std::max(hi, v);
  }
  const uintptr_t t = reinterpret_cast<uintptr_t>(a.table), d = reinterpret_cast<uintptr_t>(a.dst);
  if (op != kGatherCopy)
    ++g_counts.unemulated;
  const GatherArgs k = a;
  return set_last(enqueue_kernel(
      s, "row gather",
      {{t + static_cast<uintptr_t>(lo * row_bytes), t + static_cast<uintptr_t>((hi + 1) * row_bytes)},
       {ix, ix + static_cast<uintptr_t>(rows * iw)}},
      {d, d + static_cast<uintptr_t>(static_cast<int64_t>(a.work) * nbo)},
      [k, op, nbi, nbo, iw] {
        for (uint32_t i = 0; i < k.work; ++i) {
          const uint32_t r = i / k.row_items, j = i - r * k.row_items;
          const int64_t row = iw == 8 ? reinterpret_cast<const int64_t *>(k.idx)[r]
                                      : reinterpret_cast<const int32_t *>(k.idx)[r];
          const uint8_t *from = k.table + (row * k.row_items + j) * nbi;
          if (op == kGatherCopy)
            std::memcpy(k.dst + static_cast<int64_t>(i) * nbo, from, static_cast<size_t>(nbi));
          else
            std::memset(k.dst + static_cast<int64_t>(i) * nbo, 0, static_cast<size_t>(nbo));
        }
      }));
}

hipError_t copy16_launch(const void *src, void *dst, uint32_t n16, int /*items*/, hipStream_t s) {
  const uintptr_t sp = reinterpret_cast<uintptr_t>(src), dp = reinterpret_cast<uintptr_t>(dst);
  const size_t n = static_cast<size_t>(n16) * 16;
  std::lock_guard<std::mutex> g(g_mu);
  return set_last(enqueue_kernel(s, "copy16", {{sp, sp + n}}, {dp, dp + n},
                                 [src, dst, n] { std::memcpy(dst, src, n); }));
}

// The static state of noalloc.hip: the scratch as a device allocation of the
// stand-in, and the event every static call on the device shares.
StaticDevice &static_device(int device) {
  static std::mutex mu; // not g_mu: the event is made through the stand-in's own calls
  static StaticDevice *state[8] = {};
  std::lock_guard<std::mutex> g(mu);
  if (device < 0 || device >= 8)
    throw Error("backend_failure", "no such device");
  if (!state[device]) {
    auto *st = new StaticDevice;
    {
      std::lock_guard<std::mutex> gm(g_mu);
      st->addr = static_cast<uint8_t *>(raw_alloc(kScratchBytes));
      g_allocs[reinterpret_cast<uintptr_t>(st->addr)] =
          Alloc{kScratchBytes, Mem::Device, device, false};
    }
    if (hipEventCreateWithFlags(&st->last, hipEventDisableTiming) != hipSuccess)
      throw Error("backend_failure", "hipEventCreateWithFlags");
    state[device] = st;
  }
  return *state[device];
}

} // namespace relx

// ------------------------------------------------------------ control

extern "C" {

void fake_configure(const fake_knobs *k) {
  std::lock_guard<std::mutex> g(g_mu);
  g_knobs = k ? *k : fake_knobs{};
  const int64_t live_d = g_counts.live_device, live_p = g_counts.live_pinned;
  g_counts = fake_counts{};
  g_counts.live_device = live_d;
  g_counts.live_pinned = live_p;
  g_rng.seed(g_knobs.seed);
}

void fake_reset(void) {
  std::lock_guard<std::mutex> g(g_mu);
  for (hipError_t &e : g_sticky)
    e = hipSuccess;
  g_acc.clear();
  g_staged.clear();
  g_violations.clear();
}

void fake_get_counts(fake_counts *out) {
  std::lock_guard<std::mutex> g(g_mu);
  *out = g_counts;
}

int fake_violation_count(void) {
  std::lock_guard<std::mutex> g(g_mu);
  return static_cast<int>(g_violations.size());
}

const char *fake_violation(int i) {
  std::lock_guard<std::mutex> g(g_mu);
  return i >= 0 && static_cast<size_t>(i) < g_violations.size() ? g_violations[static_cast<size_t>(i)].c_str()
                                                                 : "";
}

void fake_host_read(const void *p, size_t n, const char *what) {
  std::lock_guard<std::mutex> g(g_mu);
  HostAgent &h = host_tick();
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  access(lo, lo + n, false, h.vc, h.id, h.vc[static_cast<size_t>(h.id)], what);
}

void fake_register_host(const void *p, size_t n) {
  std::lock_guard<std::mutex> g(g_mu);
  g_allocs[reinterpret_cast<uintptr_t>(p)] = Alloc{n, Mem::UserHost, t_device, true};
}

void fake_unregister_host(const void *p) {
  std::lock_guard<std::mutex> g(g_mu);
  auto it = g_allocs.find(reinterpret_cast<uintptr_t>(p));
  if (it == g_allocs.end())
    return;
  const uintptr_t lo = it->first, hi = lo + it->second.bytes;
  g_acc.erase(std::remove_if(g_acc.begin(), g_acc.end(),
                             [&](const Access &a) { return a.lo < hi && lo < a.hi; }),
              g_acc.end());
  g_allocs.erase(it);
}

void fake_mark_user_pinned(const void *p) {
  std::lock_guard<std::mutex> g(g_mu);
  auto it = g_allocs.find(reinterpret_cast<uintptr_t>(p));
  if (it != g_allocs.end())
    it->second.user = true;
}

int fake_host_handoff(void) {
  std::lock_guard<std::mutex> g(g_mu);
  g_tokens.push_back(host_tick().vc);
  return static_cast<int>(g_tokens.size()) - 1;
}

void fake_host_adopt(int token) {
  std::lock_guard<std::mutex> g(g_mu);
  if (token < 0 || static_cast<size_t>(token) >= g_tokens.size())
    return;
  HostAgent &h = host_tick();
  vjoin(h.vc, g_tokens[static_cast<size_t>(token)]);
}

void fake_call_begin(void) {
  std::lock_guard<std::mutex> g(g_mu);
  ++t_call;
}

void fake_shutdown(void) {
  std::vector<ihipStream_t *> all;
  {
    std::unique_lock<std::mutex> lk(g_mu);
    all = g_streams;
    for (ihipStream_t *s : all)
      s->stop = true;
    g_cv.notify_all();
  }
  for (ihipStream_t *s : all)
    s->worker.join();
}
}
