// k-means with the reference's interface (include/quiver/quantizer.h:47-58). The control flow
// (subsample, random initialization, double-precision centroid sums, empty-cluster splitting)
// runs on the host with the reference's random engine; every assignment step is one call of the
// device's exact nearest-centroid kernel (qvh_points_nearest), so the centroids come out
// bit-identical to the reference's.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "quiver/common.h"
#include "quiver/thread_pool.h"

namespace quiver {

struct KMeansParams {
  std::size_t k = 256;
  std::size_t iterations = 25;
  /// Training is subsampled to at most k * max_points_per_centroid points.
  std::size_t max_points_per_centroid = 256;
  std::uint64_t seed = 1234;
};

/// Lloyd's k-means. Returns k x dim row-major centroids. Requires n >= k.
std::vector<float> kmeans(const float* vectors, std::size_t n, std::size_t dim,
                          const KMeansParams& params, ThreadPool* pool = nullptr);

}  // namespace quiver
