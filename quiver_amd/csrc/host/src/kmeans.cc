#include <algorithm>
#include <cstring>
#include <memory>
#include <numeric>
#include <random>

#include "device_util.h"
#include "quiver/quantizer.h"

namespace quiver {

namespace {
struct PointsDeleter {
  void operator()(qvh_points* p) const noexcept { qvh_points_destroy(p); }
};
}  // namespace

// Steps and random draws as in the reference's kmeans (src/product_quantizer.cc:29-117), which
// the bit-identical result requires: subsample by a partial Fisher-Yates over rng() % (n - i),
// initialize from k distinct points the same way, then per iteration assign (on the device),
// average in double, and split each empty cluster off a donor drawn with probability
// proportional to its size.
std::vector<float> kmeans(const float* vectors, std::size_t n, std::size_t dim,
                          const KMeansParams& params, ThreadPool* pool) {
  const std::size_t k = params.k;
  QUIVER_CHECK(k > 0 && dim > 0, "kmeans: k and dim must be positive");
  QUIVER_CHECK(n >= k, "kmeans: need at least k=" + std::to_string(k) + " training points, got " +
                           std::to_string(n));
  QUIVER_CHECK(k <= 0xFFFFFFFFull && dim <= 0xFFFFFFFFull, "kmeans: k or dim too large");
  ThreadPool& tp = pool ? *pool : ThreadPool::global();
  std::mt19937_64 rng(params.seed);

  const float* x = vectors;
  std::vector<float> sample;
  const std::size_t cap = k * std::max<std::size_t>(1, params.max_points_per_centroid);
  if (n > cap) {
    std::vector<std::size_t> order(n);
    std::iota(order.begin(), order.end(), std::size_t{0});
    for (std::size_t i = 0; i < cap; ++i) std::swap(order[i], order[i + rng() % (n - i)]);
    sample.resize(cap * dim);
    for (std::size_t i = 0; i < cap; ++i) {
      std::memcpy(sample.data() + i * dim, vectors + order[i] * dim, dim * sizeof(float));
    }
    x = sample.data();
    n = cap;
  }

  std::vector<float> cent(k * dim);
  {
    std::vector<std::size_t> order(n);
    std::iota(order.begin(), order.end(), std::size_t{0});
    for (std::size_t i = 0; i < k; ++i) {
      std::swap(order[i], order[i + rng() % (n - i)]);
      std::memcpy(cent.data() + i * dim, x + order[i] * dim, dim * sizeof(float));
    }
  }

  qvh_points* raw = nullptr;
  internal::qvh_check(qvh_points_create(x, n, static_cast<std::uint32_t>(dim), &raw), "kmeans");
  std::unique_ptr<qvh_points, PointsDeleter> points(raw);

  std::vector<std::uint32_t> assign(n);
  std::vector<double> sums(k * dim);
  std::vector<std::size_t> counts(k);
  for (std::size_t iter = 0; iter < params.iterations; ++iter) {
    internal::qvh_check(qvh_points_nearest(points.get(), cent.data(), static_cast<std::uint32_t>(k), 0,
                                           assign.data()),
                        "kmeans assignment");
    std::fill(counts.begin(), counts.end(), std::size_t{0});
    for (std::size_t i = 0; i < n; ++i) ++counts[assign[i]];
    // Per (cluster, dimension) the points are added in index order; chunks split dimensions.
    tp.parallel_for(dim, 8, [&](std::size_t jb, std::size_t je) {
      for (std::size_t c = 0; c < k; ++c)
        for (std::size_t j = jb; j < je; ++j) sums[c * dim + j] = 0.0;
      for (std::size_t i = 0; i < n; ++i) {
        const std::size_t c = assign[i];
        for (std::size_t j = jb; j < je; ++j) sums[c * dim + j] += static_cast<double>(x[i * dim + j]);
      }
    });
    for (std::size_t c = 0; c < k; ++c) {
      if (counts[c] == 0) continue;
      for (std::size_t j = 0; j < dim; ++j) {
        cent[c * dim + j] = static_cast<float>(sums[c * dim + j] / static_cast<double>(counts[c]));
      }
    }
    for (std::size_t c = 0; c < k; ++c) {
      if (counts[c] != 0) continue;
      std::size_t donor = 0;
      for (;;) {
        donor = rng() % k;
        const double share =
            static_cast<double>(counts[donor]) / static_cast<double>(n) * static_cast<double>(k);
        if (share > std::uniform_real_distribution<double>(0.0, 1.0)(rng)) break;
      }
      constexpr float kEps = 1.0f / 1024.0f;
      for (std::size_t j = 0; j < dim; ++j) {
        const float v = cent[donor * dim + j];
        const float sign = (j % 2 == 0) ? 1.0f : -1.0f;
        cent[c * dim + j] = v * (1.0f + sign * kEps);
        cent[donor * dim + j] = v * (1.0f - sign * kEps);
      }
      counts[c] = counts[donor] / 2;
      counts[donor] -= counts[c];
    }
  }
  return cent;
}

}  // namespace quiver
