// hip_fake.h - control interface of the CPU stand-in for the HIP runtime
// (tests/native/hip_fake.cpp) that librelx's host sources are linked against
// in the CPU tests.
//
// The stand-in implements the HIP calls the host sources make (memory,
// streams, events, copies, pointer attributes) and the four device entry
// points they launch through (relx::launch_box, relx::gather_launch,
// relx::copy16_launch, relx::static_device). Streams are worker threads
// that run their operations in order; events complete when their stream
// reaches them. Device memory is host memory.
//
// On top of that it keeps, for every operation, the vector clock HIP's
// ordering rules give it at the moment it is enqueued (stream order, events
// recorded and waited on, host synchronization), and checks every access to
// device memory, page-locked memory and registered host buffers against the
// earlier conflicting accesses: a read or write that is not ordered after an
// earlier write (or a write not ordered after an earlier read) of the same
// bytes is a violation. The check depends only on the order of the calls,
// not on how the worker threads happen to be scheduled.
//
// Fault knobs make the n-th call of a kind fail when it is made, or the n-th
// operation fail when its stream runs it (a sticky device error that every
// later synchronization reports, as a device fault does), make
// synchronization report an unknown outcome, and delay operations.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

extern "C" {

typedef struct fake_knobs {
  int fail_malloc_at;       // n-th hipMalloc fails (hipErrorOutOfMemory); 0 = never
  int fail_host_malloc_at;  // n-th hipHostMalloc fails (hipErrorOutOfMemory)
  int fail_copy_at;         // n-th hipMemcpyAsync is refused when submitted
  int fail_copy_async_at;   // n-th hipMemcpyAsync faults on its stream (sticky)
  int fail_launch_at;       // n-th kernel launch is refused when submitted
  int fail_kernel_async_at; // n-th kernel faults on its stream (sticky)
  int fail_record_at;       // n-th hipEventRecord is refused
  int fail_wait_at;         // n-th hipStreamWaitEvent is refused
  int fail_sync_at;         // n-th stream/event synchronize reports hipErrorUnknown
  int sync_unknown;         // every stream/event synchronize reports hipErrorUnknown
  int delay_copy_us;        // each copy waits this long on its stream before it runs
  int delay_kernel_us;      // each kernel waits this long on its stream before it runs
  int jitter;               // 1: delays are uniform in [0, delay] instead of fixed
  uint32_t seed;            // jitter seed
  int device_count;         // devices hipGetDeviceCount reports (default 1)
} fake_knobs;

typedef struct fake_counts {
  int64_t mallocs, host_mallocs, copies, launches, records, waits, syncs;
  int64_t frees, host_frees, live_device, live_pinned;
  int64_t unemulated; // kernels whose value stages the stand-in does not run
  int64_t zero_copy;  // kernels that read the library's page-locked staging
} fake_counts;

// Set the knobs and reset the call counters they count against.
void fake_configure(const fake_knobs *k);
// Clear sticky errors, recorded accesses and violations (streams must be idle).
void fake_reset(void);
void fake_get_counts(fake_counts *out);

int fake_violation_count(void);
const char *fake_violation(int i);

// The calling thread reads [p, p + n) now: it must be ordered after every
// recorded write of those bytes.
void fake_host_read(const void *p, size_t n, const char *what);
// Track (or stop tracking) accesses to a pageable host buffer of the caller.
void fake_register_host(const void *p, size_t n);
void fake_unregister_host(const void *p);
// Page-locked buffers the caller owns (not the library's staging): a copy
// from them does not count as a host write made just before it.
void fake_mark_user_pinned(const void *p);

// Ordering between host threads (thread start and join, or any hand-off):
// the thread that hands over takes a token of everything it has done so
// far; the thread that takes over adopts it.
int fake_host_handoff(void);
void fake_host_adopt(int token);

// The calling thread starts a library call. The library stages a zero-copy
// chunk on the host once and then launches the chunk's kernels (one per box
// of its program) against it; the stand-in records that staging as a host
// write of the slot at the first kernel of a call that reads the slot for a
// destination, not again at the later kernels of the same chunk.
void fake_call_begin(void);

// Stop every stream's worker (streams of quarantined contexts included).
void fake_shutdown(void);
}
