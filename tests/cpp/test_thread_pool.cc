// quiver::ThreadPool semantics (include/quiver/thread_pool.h:14-57 of the reference): every item of
// [0, n) runs exactly once, in chunks of at most `grain` when the loop is spread over threads, or as
// one call fn(0, n) when it runs inline (one thread, n <= grain, or inside a chunk), as the
// reference's parallel_for does (src/thread_pool.cc:95-104); a chunk's exception
// reaches the caller (the first one, and the pool stays usable); a loop issued inside a chunk runs
// inline; concurrent callers are serialized. Exits non-zero on a failure.
#include <atomic>
#include <cstdio>
#include <stdexcept>
#include <thread>
#include <vector>

#include "quiver/thread_pool.h"

namespace {
int g_failures = 0;
#define EXPECT(cond)                                                           \
  do {                                                                         \
    if (!(cond)) {                                                             \
      std::printf("expectation failed: %s (line %d)\n", #cond, __LINE__);     \
      ++g_failures;                                                            \
    }                                                                          \
  } while (0)
}  // namespace

int main() {
  for (std::size_t threads : {1u, 2u, 5u, 16u}) {
    quiver::ThreadPool pool(threads);
    EXPECT(pool.num_threads() == threads);
    for (std::size_t n : {0u, 1u, 7u, 1000u, 100003u}) {
      for (std::size_t grain : {0u, 1u, 3u, 64u, 5000u}) {
        std::vector<std::atomic<int>> hits(n);
        std::atomic<std::size_t> oversized{0};
        pool.parallel_for(n, grain, [&](std::size_t b, std::size_t e) {
          const bool inline_run = threads == 1 || n <= (grain == 0 ? 1 : grain);
          if (inline_run ? (b != 0 || e != n) : e - b > (grain == 0 ? 1 : grain)) ++oversized;
          for (std::size_t i = b; i < e; ++i) ++hits[i];
        });
        bool once = true;
        for (auto& h : hits) once = once && h.load() == 1;
        EXPECT(once && oversized == 0);
      }
    }
    // The first exception reaches the caller; later loops run normally.
    bool caught = false;
    try {
      pool.parallel_for(10000, 10, [](std::size_t b, std::size_t) {
        if (b % 1000 == 0) throw std::runtime_error("chunk failed");
      });
    } catch (const std::runtime_error& e) {
      caught = std::string(e.what()) == "chunk failed";
    }
    EXPECT(caught);
    std::atomic<std::size_t> sum{0};
    pool.parallel_for(1000, 7, [&](std::size_t b, std::size_t e) {
      for (std::size_t i = b; i < e; ++i) sum += i;
    });
    EXPECT(sum == 999 * 1000 / 2);
    // A nested loop runs inline on the chunk's thread.
    std::atomic<int> nested_foreign{0};
    pool.parallel_for(64, 1, [&](std::size_t, std::size_t) {
      const auto me = std::this_thread::get_id();
      pool.parallel_for(100, 1, [&](std::size_t, std::size_t) {
        if (std::this_thread::get_id() != me) ++nested_foreign;
      });
    });
    EXPECT(nested_foreign == 0);
    // Concurrent callers.
    std::atomic<std::size_t> total{0};
    std::vector<std::thread> callers;
    for (int c = 0; c < 4; ++c) {
      callers.emplace_back([&] {
        for (int r = 0; r < 50; ++r) pool.parallel_for(257, 8, [&](std::size_t b, std::size_t e) { total += e - b; });
      });
    }
    for (auto& t : callers) t.join();
    EXPECT(total == 4u * 50u * 257u);
  }
  EXPECT(quiver::ThreadPool::global().num_threads() >= 1);
  std::printf("%s\n", g_failures == 0 ? "thread pool ok" : "thread pool FAILED");
  return g_failures == 0 ? 0 : 1;
}
