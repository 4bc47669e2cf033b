// workers.h - the host worker pool of the staging pipeline (plain C++, no
// HIP: the CPU tests build it alone under ThreadSanitizer).
#pragma once

#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

namespace relx {

// Persistent worker threads; parallel_for splits [0, n) into contiguous
// ranges (no smaller than `grain`), range i belonging to thread i (the
// calling thread is thread 0). Each range is claimed once, by its owner or,
// when the owner has not woken by the time the caller finished its own, by
// the caller: a worker that sleeps through a job (descheduled, or slow to
// wake) then costs one range of time instead of its wake-up latency.
// Between jobs the workers (and the caller, waiting for them) spin for a
// short while before sleeping: a pipeline hands them one job per chunk, and
// waking sleeping threads costs tens of microseconds per job.
class Workers {
public:
  explicit Workers(unsigned threads);
  ~Workers();
  unsigned size() const { return static_cast<unsigned>(threads_.size()) + 1; }
  // At most `max_parts` ranges (0: one per thread of the pool).
  void parallel_for(int64_t n, int64_t grain, const std::function<void(int64_t, int64_t)> &fn,
                    unsigned max_parts = 0);

private:
  void loop(unsigned id);
  // Runs range i if nobody has claimed it yet in this job.
  void run_range(size_t i);
  std::vector<std::thread> threads_;
  std::mutex mu_;
  std::condition_variable go_, done_;
  const std::function<void(int64_t, int64_t)> *fn_ = nullptr;
  std::vector<std::pair<int64_t, int64_t>> ranges_;
  std::unique_ptr<std::atomic<int>[]> claimed_; // per range: 0 free, 1 claimed
  std::atomic<int64_t> parts_{0}, completed_{0};
  std::atomic<uint64_t> generation_{0};
  std::atomic<bool> stop_{false};
};

} // namespace relx
