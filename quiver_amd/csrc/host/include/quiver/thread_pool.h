// Fork-join pool for the host-side work around the device calls (filter materialization, label
// mapping, k-means centroid updates), with the reference's interface and semantics
// (include/quiver/thread_pool.h:14-57): the caller participates, nested parallel_for calls run
// inline, and the first exception thrown by a chunk is rethrown to the caller.
#pragma once

#include <cstddef>
#include <functional>
#include <memory>
#include <mutex>
#include <semaphore>
#include <vector>

namespace quiver {

class ThreadPool {
 public:
  using RangeFn = std::function<void(std::size_t begin, std::size_t end)>;

  /// `num_threads` counts the calling thread; 0 means std::thread::hardware_concurrency().
  explicit ThreadPool(std::size_t num_threads = 0);
  ~ThreadPool();
  ThreadPool(const ThreadPool&) = delete;
  ThreadPool& operator=(const ThreadPool&) = delete;

  std::size_t num_threads() const noexcept { return helpers_.size() + 1; }

  /// Runs fn over [0, n) in chunks of at most `grain` items and blocks until all finish.
  void parallel_for(std::size_t n, std::size_t grain, const RangeFn& fn);

  /// Process-wide pool sized to the machine.
  static ThreadPool& global();

 private:
  struct Loop;    // the shared state of one parallel_for call
  struct Helper;  // a helper thread and the semaphore that hands it a loop

  void serve(Helper& helper);
  void stop_helpers() noexcept;

  std::vector<std::unique_ptr<Helper>> helpers_;
  std::mutex calls_;                    // one parallel_for at a time per pool
  std::binary_semaphore finished_{0};  // released by the last helper to leave a loop
};

}  // namespace quiver
