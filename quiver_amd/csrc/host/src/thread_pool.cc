#include "quiver/thread_pool.h"

#include <algorithm>
#include <atomic>

namespace quiver {
namespace {
// Set while this thread executes a chunk of some pool: nested loops then run inline.
thread_local bool t_in_chunk = false;
}  // namespace

struct ThreadPool::Task {
  const RangeFn* fn = nullptr;
  std::size_t n = 0, grain = 1;
  std::atomic<std::size_t> cursor{0};
  std::atomic<bool> failed{false};
  std::mutex err_mu;
  std::exception_ptr error;
};

ThreadPool::ThreadPool(std::size_t num_threads) {
  if (num_threads == 0) num_threads = std::max<std::size_t>(1, std::thread::hardware_concurrency());
  try {
    for (std::size_t i = 1; i < num_threads; ++i) threads_.emplace_back([this] { worker(); });
  } catch (...) {
    {
      std::lock_guard<std::mutex> lock(mu_);
      stopping_ = true;
    }
    wake_.notify_all();
    for (auto& t : threads_) t.join();
    throw;
  }
}

ThreadPool::~ThreadPool() {
  {
    std::lock_guard<std::mutex> lock(mu_);
    stopping_ = true;
  }
  wake_.notify_all();
  for (auto& t : threads_) t.join();
}

ThreadPool& ThreadPool::global() {
  static ThreadPool pool;
  return pool;
}

void ThreadPool::drain(Task& task) noexcept {
  const bool outer = t_in_chunk;
  t_in_chunk = true;
  while (!task.failed.load(std::memory_order_relaxed)) {
    const std::size_t b = task.cursor.fetch_add(task.grain, std::memory_order_relaxed);
    if (b >= task.n) break;
    try {
      (*task.fn)(b, std::min(task.n, b + task.grain));
    } catch (...) {
      std::lock_guard<std::mutex> lock(task.err_mu);
      if (!task.error) task.error = std::current_exception();
      task.failed.store(true, std::memory_order_relaxed);
    }
  }
  t_in_chunk = outer;
}

void ThreadPool::worker() {
  std::uint64_t seen = 0;
  std::unique_lock<std::mutex> lock(mu_);
  for (;;) {
    wake_.wait(lock, [&] { return stopping_ || epoch_ != seen; });
    if (stopping_) return;
    seen = epoch_;
    Task* task = task_;
    lock.unlock();
    drain(*task);
    lock.lock();
    if (--busy_ == 0) idle_.notify_one();
  }
}

void ThreadPool::parallel_for(std::size_t n, std::size_t grain, const RangeFn& fn) {
  if (n == 0) return;
  grain = std::max<std::size_t>(grain, 1);
  if (threads_.empty() || n <= grain || t_in_chunk) {
    fn(0, n);
    return;
  }
  std::lock_guard<std::mutex> submit(submit_);
  Task task;
  task.fn = &fn;
  task.n = n;
  task.grain = grain;
  {
    std::lock_guard<std::mutex> lock(mu_);
    task_ = &task;
    busy_ = threads_.size();
    ++epoch_;
  }
  wake_.notify_all();
  drain(task);
  {
    std::unique_lock<std::mutex> lock(mu_);
    idle_.wait(lock, [&] { return busy_ == 0; });
    task_ = nullptr;
  }
  if (task.error) std::rethrow_exception(task.error);
}

}  // namespace quiver
