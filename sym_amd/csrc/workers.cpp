// workers.cpp - the host worker pool (see workers.h).
#include "workers.h"

#include <immintrin.h>

#include <algorithm>
#include <chrono>

namespace relx {

namespace {

// How long an idle worker, or a caller waiting for its workers, spins
// before blocking.
constexpr auto kSpin = std::chrono::microseconds(200);

template <class Pred> bool spin_until(Pred done) {
  const auto t0 = std::chrono::steady_clock::now();
  for (unsigned i = 0; !done(); ++i) {
    _mm_pause();
    if ((i & 63) == 63 && std::chrono::steady_clock::now() - t0 > kSpin)
      return done();
  }
  return true;
}

} // namespace

Workers::Workers(unsigned threads) {
  const unsigned total = std::max(1u, threads);
  claimed_.reset(new std::atomic<int>[total]);
  ranges_.assign(total, {0, 0});
  for (unsigned i = 0; i < total; ++i)
    claimed_[i].store(1, std::memory_order_relaxed);
  for (unsigned i = 1; i < total; ++i)
    threads_.emplace_back([this, i] { loop(i); });
}

Workers::~Workers() {
  {
    std::lock_guard<std::mutex> g(mu_);
    stop_.store(true);
  }
  go_.notify_all();
  for (auto &t : threads_)
    t.join();
}

void Workers::run_range(size_t i) {
  // The claim (acquire) orders the range and function reads after the
  // caller's reset of this flag (release), which follows their writes.
  if (claimed_[i].exchange(1, std::memory_order_acq_rel) != 0)
    return;
  const std::pair<int64_t, int64_t> r = ranges_[i];
  if (r.second > r.first)
    (*fn_)(r.first, r.second);
  if (completed_.fetch_add(1, std::memory_order_acq_rel) + 1 ==
      parts_.load(std::memory_order_relaxed)) {
    std::lock_guard<std::mutex> g(mu_);
    done_.notify_one();
  }
}

void Workers::loop(unsigned id) {
  uint64_t seen = 0;
  for (;;) {
    auto ready = [&] { return stop_.load() || generation_.load(std::memory_order_acquire) != seen; };
    if (!spin_until(ready)) {
      std::unique_lock<std::mutex> g(mu_);
      go_.wait(g, ready);
    }
    if (stop_.load())
      return;
    seen = generation_.load(std::memory_order_acquire);
    if (static_cast<int64_t>(id) < parts_.load(std::memory_order_acquire))
      run_range(id);
  }
}

void Workers::parallel_for(int64_t n, int64_t grain,
                           const std::function<void(int64_t, int64_t)> &fn, unsigned max_parts) {
  const unsigned total = max_parts ? std::min(max_parts, size()) : size();
  const int64_t parts =
      std::max<int64_t>(1, std::min<int64_t>(total, n / std::max<int64_t>(1, grain)));
  if (parts <= 1 || threads_.empty()) {
    if (n > 0)
      fn(0, n);
    return;
  }
  {
    // Every range of the previous job has completed, so no thread is inside
    // run_range: the ranges, the function and the flags can be rewritten.
    std::lock_guard<std::mutex> g(mu_);
    for (int64_t i = 0; i < parts; ++i)
      ranges_[static_cast<size_t>(i)] = {n * i / parts, n * (i + 1) / parts};
    fn_ = &fn;
    completed_.store(0, std::memory_order_relaxed);
    parts_.store(parts, std::memory_order_relaxed);
    for (int64_t i = 0; i < parts; ++i)
      claimed_[static_cast<size_t>(i)].store(0, std::memory_order_release);
    generation_.fetch_add(1, std::memory_order_release);
  }
  go_.notify_all();
  for (int64_t i = 0; i < parts; ++i) // own range first, then any still unclaimed
    run_range(static_cast<size_t>(i));
  auto finished = [&] { return completed_.load(std::memory_order_acquire) == parts; };
  if (!spin_until(finished)) {
    std::unique_lock<std::mutex> g(mu_);
    done_.wait(g, finished);
  }
}

} // namespace relx
