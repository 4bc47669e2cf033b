// runtime.h - internal declarations shared by program.cpp, runtime.cpp,
// indexed.cpp and capi.cpp.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/relx.h"
#include "plan.h"
#include "program.h"
#include "workers.h"

namespace relx {

// Makes `dev` the current device for a scope, restoring the previous one.
struct DeviceScope {
  int prev = -1;
  explicit DeviceScope(int dev) {
    if (hipGetDevice(&prev) != hipSuccess)
      prev = -1;
    if (prev != dev)
      (void)hipSetDevice(dev);
  }
  ~DeviceScope() {
    int cur;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev)
      (void)hipSetDevice(prev);
  }
  DeviceScope(const DeviceScope &) = delete;
  DeviceScope &operator=(const DeviceScope &) = delete;
};

// One value stage as host scalars (reference StageArithmetic,
// libreloc/include/reloc/TypedExecute.h:52-68).
struct HostStage {
  uint8_t op = 0;
  uint32_t in_width = 0, out_width = 0;
  std::vector<float> scale, inv; // inv = fl32(1/scale) for quantize
  std::vector<int32_t> zero_point{0};
  uint8_t mode = kChanNone;
  int dim = 0;
  int64_t len = 1;
  std::vector<ChanToken> tokens; // kChanExpr, symbols resolved
};

struct Prepared {
  std::vector<HostStage> stages;
  std::vector<int64_t> res_strides;
};

struct DeviceProgram {
  int family = kFamGeneric;
  const char *kernel = "generic";
  uint32_t boundary = 0;
  KArgs base;
  int64_t wire_elems = 0, wire_bytes = 0, dst_elems = 0;
  int chunk_axis = -1;
  int64_t chunk_stride = 0, chunk_align = 1;
  int qa = -1, ca = -1; // transpose: source-inner (destination row) and destination-inner axes
  std::vector<float> pf;
  std::vector<int32_t> pi;
};

// Division by a runtime constant d >= 1 for 32-bit numerators (FastDiv).
FastDiv make_div(int64_t d);
void prepare_stages(const Bound &b, Prepared &p);
bool fill_at(const Bound &b, const Prepared &p, uint32_t to, uint64_t &bits);
uint64_t host_apply(const HostStage &s, uint64_t x, int64_t c);
std::unique_ptr<DeviceProgram> build_program(const Bound &b, const Prepared &p, uint32_t k);
std::vector<KArgs> box_launches(const DeviceProgram &dp, int64_t v0, int64_t v1, bool first,
                                bool last);
// Launches covering padded coordinates [plo, phi) of one destination axis
// (the whole box when axis < 0).
std::vector<KArgs> axis_launches(const DeviceProgram &dp, int axis, int64_t plo, int64_t phi);
// Launches for one coordinate of each axis before `axis` (fixed[0..axis))
// and padded coordinates [plo, phi) of `axis`.
std::vector<KArgs> prefix_launches(const DeviceProgram &dp, const int64_t *fixed, int axis,
                                   int64_t plo, int64_t phi);
// Coordinates a box along axis i must keep together (0: never split).
int64_t axis_align(const DeviceProgram &dp, int i);
// Launch boxes (verified first when RELX_VERIFY_LAUNCHES is set, their
// source reads inside wire elements [wire_lo, wire_hi), wire_hi < 0: all).
int64_t launch_all(const DeviceProgram &dp, std::vector<KArgs> launches, const void *src,
                   void *dst, const float *pf, const int32_t *pi, int32_t *status, hipStream_t s,
                   int64_t wire_lo = 0, int64_t wire_hi = -1);
// Launch the program over valid chunk-axis coordinates [v0, v1) (the whole
// box when it has no chunk axis); returns the number of kernel launches.
int64_t launch_program(const DeviceProgram &dp, int64_t v0, int64_t v1, bool first, bool last,
                       const void *src, void *dst, const float *pf, const int32_t *pi,
                       int32_t *status, hipStream_t s);
hipError_t launch_box(int family, const KArgs &a, int32_t *status, hipStream_t s);
// Host-side check that one launch stays inside the wire and the result, with
// aligned vectors and parameter indices inside their tables (throws Error).
// Its source reads must lie in wire elements [wire_lo, wire_hi) (wire_hi < 0:
// the whole wire).
void verify_launch(const DeviceProgram &dp, const KArgs &a, int64_t wire_lo = 0,
                   int64_t wire_hi = -1);

// Chunk schedule of one program: `units` valid coordinates of the chunk axis
// (1 without one), `per_chunk` per chunk, wire/source bytes per unit.
struct ChunkPlan {
  int64_t units, per_chunk, unit_wire, unit_src;
};
// Default chunk bytes for a transfer of `total` bytes, measured on the
// MI355X's PCIe link with chunks alternating over two copy streams: staged
// uploads a quarter of the wire within [2, 8] MiB, direct DMA half of it
// within [32, 64] MiB; device-to-host into pinned memory a quarter of the
// result within [16, 32] MiB, into pageable memory an eighth within [4, 8] MiB.
int64_t default_chunk_bytes(int64_t total, bool h2d, bool direct);
uint32_t source_width(const Bound &b);
ChunkPlan chunk_plan(const DeviceProgram &dp, uint32_t src_width, int64_t chunk_bytes, bool direct);

// The kernel launches of an upload each cover a batch of landed chunks. A
// launch streams at the HBM rate only from a few hundred MB up (C5's
// permute on cold HBM: 50 MB per launch at 0.61 of peak, 403 MB at 0.78,
// 805 MB at 0.80), while a chunk's copy takes far longer than its share of
// the kernel, so a batch takes chunks until it holds kKernelBatchBytes of
// wire. A member keeps at least four batches, so that the last one, which
// runs after the last copy, stays short.
// The last chunk is a batch of its own when batches take several chunks:
// its kernel is what runs after the last copy lands.
constexpr int64_t kKernelBatchBytes = int64_t{512} << 20;
struct KernelBatches {
  int64_t units, per; // chunk-axis units, units per batch (whole chunks)
  int64_t last;       // first unit of the last chunk when it is a batch of its own, else units
  int64_t end(int64_t k0) const {
    const int64_t e = std::min(units, k0 + per);
    return k0 < last && e > last ? last : e;
  }
};
KernelBatches kernel_batches(const ChunkPlan &p);


// Host staging transform: source elements [e0, e1) at boundary 0 -> wire
// elements at boundary `k` (leading per-tensor stages applied elementwise).
void host_transform(const Prepared &p, uint32_t k, uint32_t src_width, const void *src, void *dst,
                    int64_t e0, int64_t e1);

// ------------------------------------------------------------ handles

struct BoundHandle {
  std::unique_ptr<Bound> bound;
  Prepared prep;
  std::mutex mu;
  std::map<uint32_t, std::unique_ptr<DeviceProgram>> programs; // by wire boundary
  struct DevParams {
    float *pf = nullptr;
    int32_t *pi = nullptr;
  };
  std::map<std::pair<int, uint32_t>, DevParams> params; // (device, boundary)
  std::map<int, void *> dev_indices;                     // indexed plans, per device
  const DeviceProgram &program(uint32_t k);
  DevParams device_params(int device, uint32_t k);
  // The bound row indices in device memory (int32 when the table has fewer
  // than 2^31 rows, else int64), uploaded once per device.
  const void *device_indices(int device);
  ~BoundHandle();
};

// ------------------------------------------------------------ indexed plans

// Vector shape of a device row gather for one table/destination alignment.
struct GatherPlan {
  int op = kGatherCopy;
  int nbi = 1, nbo = 1; // source / destination bytes per item
  int iw = 4;           // index bytes
  bool nt = false;      // streaming table loads (long rows)
  int64_t row_items = 1;
};
GatherPlan gather_plan(const Bound &b, const void *table, const void *dst);
// Launches over every selected row; `idx` holds the device indices.
std::vector<GatherArgs> gather_launches(const Bound &b, const GatherPlan &g, const void *table,
                                        void *dst, const void *idx);
// Host-side check that every gather launch stays inside the table (of
// `table_bytes`), the destination (of `dst_bytes`) and the index array.
void verify_gather(const Bound &b, const GatherPlan &g, const std::vector<GatherArgs> &launches,
                   const void *table, size_t table_bytes, const void *dst, size_t dst_bytes,
                   const void *idx);
hipError_t gather_launch(const GatherArgs &a, int op, int nbi, int iw, bool nt, hipStream_t s);
// Host staging of an indexed plan: selected elements [g0, g1) (dense
// selected-row order) gathered from the table through stages [0, k) into
// `dst`, which receives element g0 first.
void host_gather(const Bound &b, const Prepared &p, uint32_t k, const void *table, void *dst,
                 int64_t g0, int64_t g1);

// Device-to-host chunk schedule: for each of the `outer` coordinate tuples of
// the destination axes before `axis`, ranges of `per` coordinates of `axis`
// (-1: one chunk), `row` bytes per coordinate; every chunk is one contiguous
// range of the dense destination.
struct D2hPlan {
  int axis;
  int64_t outer, units, per, row;
  // axis < 0: one kernel launch, then copies of `copy_bytes` each
  int64_t copy_bytes;
};
D2hPlan d2h_plan(const DeviceProgram &dp, int64_t chunk_bytes, bool pinned);

struct Context;
// Device-resident source -> host destination (see runtime.cpp).
void execute_d2h(Context &ctx, BoundHandle &h, const void *src, size_t src_bytes, void *dst,
                 size_t dst_bytes, const relx_options &opt, relx_report *report);

// Device-resident table -> device destination: the row gather with the
// plan's cast fused, asynchronous on `stream`; returns the launch count.
int64_t index_select_device(Context &ctx, BoundHandle &h, const void *table, size_t table_bytes,
                            void *dst, size_t dst_bytes, hipStream_t stream);

// Selected rows from which an upload sends the whole table instead of the
// gathered rows (when the table is no larger than the gathered wire).
constexpr int64_t kTableUploadRows = int64_t{1} << 16;
// The upload of an indexed plan whose gathered wire is `gathered_wire` bytes
// sends its table and gathers on the device: the table is no larger, and the
// selection is long enough that the host's random row reads, not the
// transfer, would set the pace.
bool table_upload_pays(const Bound &b, int64_t gathered_wire);

// HBM copy ceiling: GB/s (bytes read + written) of a 16-byte vector copy of
// `bytes`, best of `rounds` runs of `iters` copies over rotating buffers.
double measure_device_copy(int device, size_t bytes, int iters, int rounds);

// Leading per-tensor narrowing stages applied on the host for a pageable
// source (halving PCIe bytes where a cast narrows).
uint32_t auto_host_stages(const BoundHandle &h);

// verify_launch over every launch of the chunk schedules for `chunk_bytes`
// (0: both defaults, staged and direct, in each direction) and the whole-box
// launch of the device-resident path; returns the count.
int64_t verify_launches(BoundHandle &h, uint32_t k, int64_t chunk_bytes);

// A ROCTX range on the calling thread around one host phase of the pipeline
// (the reference's TraceRange, libreloc/src/Trace.h:15-39, which its NVTX
// builds emit at libreloc/src/Pipeline.cpp:204,213). Enabled at run time by
// the environment variable RELX_TRACE=1, which opens the ROCTX library on
// first use; otherwise a range costs one branch. The name carries the chunk.
class TraceRange {
public:
  // "<name> <key>=<index>", e.g. "relx.h2d.stage chunk=3", "relx.h2d.call call=7"
  TraceRange(const char *name, int64_t index, const char *key = "chunk");
  ~TraceRange();
  TraceRange(const TraceRange &) = delete;
  TraceRange &operator=(const TraceRange &) = delete;

private:
  bool open_ = false;
};

// Kernel timing of blocking uploads (relx_ctx_time_kernels): per chunk, the
// elapsed time between events recorded before and after its launches.
struct KernelTimes {
  int64_t calls = 0, chunks = 0, launches = 0;
  double ms = 0.0;
};

#ifndef RELX_COPY_STREAMS
#define RELX_COPY_STREAMS 2
#endif
// Copy streams that take the chunks of a transfer in turn: a DMA call costs
// microseconds before its bytes move, and the next stream's call hides that
// behind the previous one's transfer. Two measured best: with three, pageable
// uploads lost 2-10% (C2 77% -> 68% of the PCIe ceiling) and pageable
// downloads 6-13%.
constexpr int kCopyStreams = RELX_COPY_STREAMS;

struct StaticDevice; // the allocation-free upload's per-device state (below)

struct Context {
  int device = 0;
  hipStream_t copies[kCopyStreams] = {};
  hipStream_t compute = nullptr;
  // The stream of chunk `chunk` when a call spreads its chunks over `ns`
  // copy streams (1 or kCopyStreams).
  hipStream_t copy_stream(int64_t chunk, int ns = kCopyStreams) const {
    return copies[static_cast<size_t>(chunk % ns)];
  }
  std::vector<void *> slots;
  size_t slot_bytes = 0;
  std::vector<hipEvent_t> slot_ev;
  std::vector<bool> slot_pending; // an event was recorded since the slot was last known idle
  std::vector<hipEvent_t> chunk_ev;
  hipEvent_t start_ev = nullptr, done_ev = nullptr;
  hipEvent_t join_ev[kCopyStreams] = {}; // one per copy stream, for joins
  uint8_t *wire = nullptr;
  size_t wire_cap = 0;
  int32_t *status = nullptr; // kStatusSlots flags, one per call in flight,
                             // then kDeviceChecks flags of device-resident calls
  uint32_t status_next = 0; // wraps
  // Device-resident element-wise launches (relx_relayout_device) run on the
  // caller's stream and return at once: each takes the next of kDeviceChecks
  // flags and records check_ev after its launch. The flag is read once that
  // event completes: when the slot comes round again, or at synchronize.
  hipEvent_t check_ev[64] = {};
  bool check_pending[64] = {};
  uint32_t check_next = 0;
  bool channel_error = false; // a resolved check found its flag set
  bool time_kernels = false;
  KernelTimes kt;
  std::vector<hipEvent_t> time_ev; // timing event pairs, reused call to call
  // The allocation-free upload: this device's static state (its copy of the
  // scratch, the event and lock its static calls share) and pinned staging
  // for the parameter tables it uploads (kScratchParamBytes, allocated
  // here).
  StaticDevice *stat = nullptr;
  uint8_t *param_stage = nullptr;
  // Parameter tables by content: a fresh binding of a plan with the same
  // tables (the same plan and parameters, bound again for the next call)
  // finds them here and uploads nothing. Each entry is one device block
  // (floats, then ints at a 256-byte offset), written once and freed with
  // the context; past kParamCacheEntries or kParamCacheBytes a bound handle
  // keeps its own copy instead.
  std::map<std::string, BoundHandle::DevParams> param_cache;
  size_t param_cache_bytes = 0;
  std::unique_ptr<Workers> workers;
  unsigned worker_threads = 0;
  // Scratch kept between calls (ring + wire arena), in bytes; negative: no
  // bound. Checked once a blocking call has completed.
  int64_t max_retained = -1;
  std::mutex mu;
  int64_t calls = 0, failures = 0;
  // The last call returned before its work completed (a submitted group or
  // no_wait): done_ev marks its end, and the next call that reuses the wire
  // arena orders its streams after it.
  bool unsynced = false;
  std::thread::id last_thread; // the thread of the previous pipeline call
  bool quarantined = false;
  bool closed = false;
  ~Context(); // frees the status flags (the rest goes in destroy_context)
};

// The allocation-free upload's device scratch (noalloc.hip): one file-scope
// array of kScratchBytes on each GPU the library runs on, held until the
// process ends. The wire is staged in its first kScratchWireBytes; the
// parameter tables (floats, then ints) take the two halves of the last
// kScratchParamBytes.
constexpr size_t kScratchBytes = size_t{64} << 20;
constexpr size_t kScratchParamBytes = size_t{1} << 20;
constexpr size_t kScratchWireBytes = kScratchBytes - kScratchParamBytes;
constexpr size_t kParamStageHalf = kScratchParamBytes / 2;
// One device's share of the allocation-free upload, kept until the process
// ends. Every context on the device uses it: a static call holds `mu` from
// its checks to its return, its copies wait for `last` (recorded at the end
// of the previous static call on the device, from any context) before they
// write the scratch, and it records `last` again at its end. So calls from
// several contexts or threads on one GPU take the scratch in turn, also
// after a call that returned early (no_wait).
struct StaticDevice {
  uint8_t *addr = nullptr; // this device's copy of the scratch
  hipEvent_t last = nullptr;
  std::mutex mu;
};
// `device`'s static state: the scratch address from hipGetSymbolAddress and
// the event, made on the first call for the device (a context's creation);
// call with `device` current.
StaticDevice &static_device(int device);

// Bounds of Context::param_cache.
constexpr size_t kParamCacheEntries = 4096;
constexpr size_t kParamCacheBytes = size_t{16} << 20;

// Release ring and wire arena until what the context keeps fits its
// max_retained; a no-op while a call may still be running.
void trim_retained(Context &ctx);

constexpr uint32_t kStatusSlots = 1024;
constexpr uint32_t kDeviceChecks = 64; // size of Context::check_ev

// An asynchronous call's completion: an event recorded after its last kernel
// and the status flag its element-wise kernels report into. Holds the context
// so the flag outlives a close.
struct Completion {
  std::shared_ptr<Context> ctx;
  hipEvent_t ev = nullptr;
  int32_t *status = nullptr;
  bool generic = false;
  bool checked = false;
};

// Wait for a completion, then check its status flag ("channel_out_of_range").
void completion_wait(Completion &c);
// The status check alone, once the completion's event has completed.
void completion_check(Completion &c);

} // namespace relx
