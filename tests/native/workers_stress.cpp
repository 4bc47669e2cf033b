// Stress test of relx::Workers (sym_amd/csrc/workers.cpp), built with g++
// under ThreadSanitizer by tests/test_workers.py: many jobs in a row, jobs of
// every size, workers that are slow to start (the caller then claims their
// ranges), workers that sleep between jobs, and jobs that cap their ranges
// below the pool's size (the other workers stay idle); every element of
// every job must be visited exactly once.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <random>
#include <thread>
#include <vector>

#include "workers.h"

int main() {
  std::mt19937 rng(20260710);
  for (unsigned threads : {1u, 2u, 3u, 8u, 13u}) {
    relx::Workers w(threads);
    std::vector<std::atomic<int>> hits(1 << 14);
    for (int job = 0; job < 400; ++job) {
      const int64_t n = static_cast<int64_t>(rng() % (1u << 14));
      const int64_t grain = 1 + static_cast<int64_t>(rng() % 512);
      const int mode = job % 4; // 0 plain, 1 slow start, 2 uneven work, 3 a pause first
      for (int64_t i = 0; i < n; ++i)
        hits[static_cast<size_t>(i)].store(0, std::memory_order_relaxed);
      if (mode == 3)
        std::this_thread::sleep_for(std::chrono::microseconds(300)); // workers go to sleep
      // every third job caps its ranges at 1..threads+1 (0: one per thread)
      const unsigned cap = job % 3 == 2 ? 1 + static_cast<unsigned>(rng() % (threads + 1)) : 0;
      w.parallel_for(n, grain, [&](int64_t a, int64_t b) {
        if (mode == 1 && a > 0)
          std::this_thread::sleep_for(std::chrono::microseconds(50));
        for (int64_t i = a; i < b; ++i) {
          hits[static_cast<size_t>(i)].fetch_add(1, std::memory_order_relaxed);
          if (mode == 2 && (i & 1023) == 0)
            std::this_thread::yield();
        }
      }, cap);
      for (int64_t i = 0; i < n; ++i)
        if (hits[static_cast<size_t>(i)].load(std::memory_order_relaxed) != 1) {
          std::printf("threads %u job %d n %lld: element %lld visited %d times\n", threads, job,
                      static_cast<long long>(n), static_cast<long long>(i),
                      hits[static_cast<size_t>(i)].load());
          return 1;
        }
    }
  }
  std::printf("ok\n");
  return 0;
}
