#include "quiver/thread_pool.h"

#include <algorithm>
#include <atomic>
#include <exception>
#include <thread>

namespace quiver {

namespace {
// Depth of loops this thread is running chunks of (any pool): a parallel_for issued from inside a
// chunk runs inline rather than waiting for helpers that may all be busy with the outer loop.
thread_local int t_loop_depth = 0;
}  // namespace

// One parallel_for: chunks are claimed from an atomic cursor by the caller and every helper; the
// first exception wins, and once one is recorded no new chunk starts.
struct ThreadPool::Loop {
  const RangeFn& fn;
  const std::size_t n, grain;
  std::atomic<std::size_t> cursor{0};
  std::atomic<std::size_t> helpers_inside{0};
  std::atomic<bool> failed{false};
  std::once_flag error_once;
  std::exception_ptr error;

  Loop(const RangeFn& f, std::size_t count, std::size_t g) : fn(f), n(count), grain(g) {}

  void claim_chunks() noexcept {
    ++t_loop_depth;
    for (;;) {
      if (failed.load(std::memory_order_relaxed)) break;
      const std::size_t begin = cursor.fetch_add(grain, std::memory_order_relaxed);
      if (begin >= n) break;
      try {
        fn(begin, std::min(n, begin + grain));
      } catch (...) {
        std::call_once(error_once, [&] { error = std::current_exception(); });
        failed.store(true, std::memory_order_relaxed);
      }
    }
    --t_loop_depth;
  }
};

// A helper sleeps on its own semaphore; the caller of parallel_for stores the loop (or null, to
// stop it) and releases the semaphore, which orders that store before the helper reads it.
struct ThreadPool::Helper {
  std::binary_semaphore wake{0};
  Loop* loop = nullptr;
  std::thread thread;
};

ThreadPool::ThreadPool(std::size_t num_threads) {
  const std::size_t total = num_threads != 0 ? num_threads : std::max(1u, std::thread::hardware_concurrency());
  try {
    while (helpers_.size() + 1 < total) {
      auto h = std::make_unique<Helper>();
      Helper& ref = *h;
      helpers_.push_back(std::move(h));
      ref.thread = std::thread([this, &ref] { serve(ref); });
    }
  } catch (...) {
    stop_helpers();
    throw;
  }
}

ThreadPool::~ThreadPool() { stop_helpers(); }

void ThreadPool::stop_helpers() noexcept {
  for (auto& h : helpers_) {
    if (!h->thread.joinable()) continue;
    h->loop = nullptr;
    h->wake.release();
    h->thread.join();
  }
  helpers_.clear();
}

ThreadPool& ThreadPool::global() {
  static ThreadPool pool;
  return pool;
}

void ThreadPool::serve(Helper& helper) {
  for (;;) {
    helper.wake.acquire();
    Loop* loop = helper.loop;
    if (loop == nullptr) return;
    loop->claim_chunks();
    // The last helper out wakes the caller; nothing of the loop is touched after this count.
    if (loop->helpers_inside.fetch_sub(1, std::memory_order_acq_rel) == 1) finished_.release();
  }
}

void ThreadPool::parallel_for(std::size_t n, std::size_t grain, const RangeFn& fn) {
  if (n == 0) return;
  grain = std::max<std::size_t>(grain, 1);
  if (helpers_.empty() || n <= grain || t_loop_depth > 0) {
    fn(0, n);
    return;
  }
  std::lock_guard<std::mutex> one_at_a_time(calls_);
  Loop loop(fn, n, grain);
  loop.helpers_inside.store(helpers_.size(), std::memory_order_relaxed);
  for (auto& h : helpers_) {
    h->loop = &loop;
    h->wake.release();
  }
  loop.claim_chunks();
  finished_.acquire();  // every helper has left the loop
  if (loop.error) std::rethrow_exception(loop.error);
}

}  // namespace quiver
