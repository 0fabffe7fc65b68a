// Helpers shared by the host classes for calling the qvh C-ABI.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "qvh.h"
#include "quiver/common.h"
#include "quiver/filter.h"
#include "quiver/thread_pool.h"

namespace quiver::internal {

/// Throws quiver::Error carrying qvh_last_error() when a qvh call failed.
inline void qvh_check(qvh_status status, const char* what) {
  if (status != QVH_OK) {
    throw Error(std::string(what) + ": " + qvh_last_error());
  }
}

inline void check_finite(const float* v, std::size_t count) {
  bool ok = true;
  for (std::size_t i = 0; i < count; ++i) ok &= std::isfinite(v[i]);
  QUIVER_CHECK(ok, "vectors must not contain NaN or infinity");
}

/// Bitmap over ids [0, n): bit i set iff filter->contains(label_of(i)). Words are filled in
/// parallel chunks of whole words, so no two chunks touch one word.
template <class LabelOf>
std::vector<std::uint64_t> filter_bitmap(const Filter& filter, std::size_t n, LabelOf label_of,
                                         ThreadPool& pool) {
  const std::size_t words = (n + 63) / 64;
  std::vector<std::uint64_t> bits(words == 0 ? 1 : words, 0);
  pool.parallel_for(words, 256, [&](std::size_t wb, std::size_t we) {
    for (std::size_t w = wb; w < we; ++w) {
      std::uint64_t word = 0;
      const std::size_t end = std::min(n, (w + 1) * 64);
      for (std::size_t i = w * 64; i < end; ++i) {
        if (filter.contains(label_of(i))) word |= std::uint64_t{1} << (i - w * 64);
      }
      bits[w] = word;
    }
  });
  return bits;
}

}  // namespace quiver::internal
