// k-means, nearest_centroid and the product quantizer, with the reference's interface
// (include/quiver/quantizer.h:47-114).
//
// k-means runs its control flow (subsample, random initialization, double-precision centroid sums,
// empty-cluster splitting) on the host with the reference's random engine; every assignment step is
// one call of the device's exact nearest-centroid kernel (qvh_points_nearest), so the centroids
// come out bit-identical to the reference's. The reference's per-vector methods (nearest_centroid,
// ProductQuantizer::encode / decode / compute_*_table / adc / adc_batch) run on the host in the
// reference's float order and cannot fail, as the reference's noexcept versions cannot; the
// *_batch methods (no reference counterpart) run many vectors per device call (qvh_nearest_centroid,
// qvh_pq_*) with the same arithmetic and throw quiver::Error on a device failure.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

#include "quiver/common.h"
#include "quiver/thread_pool.h"

struct qvh_pq;

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

/// Index of the centroid nearest to `x` (squared L2 in the AVX2 kernels' order; the first of equal
/// ones; 0 when no distance is finite). Host code.
std::size_t nearest_centroid(const float* x, const float* centroids, std::size_t k,
                             std::size_t dim) noexcept;

/// The same for n row-major points (no reference counterpart): out[i] for point i.
void nearest_centroid_batch(const float* x, std::size_t n, const float* centroids, std::size_t k,
                            std::size_t dim, std::uint32_t* out);

/// PQ: the vector is split into `m` sub-vectors, each replaced by the id of its nearest of 256
/// sub-centroids, so a vector costs `m` bytes; distances to a query use asymmetric distance
/// computation over an m x 256 table. The codebook is kept on the host and on the device once
/// trained or set; copies share the device copy. The noexcept methods compute on the host; the
/// *_batch methods on the device, throwing quiver::Error if it fails.
class ProductQuantizer {
 public:
  static constexpr std::size_t kSubCentroids = 256;

  ProductQuantizer();
  /// `dim` must be divisible by `m`.
  ProductQuantizer(std::size_t dim, std::size_t m);
  ~ProductQuantizer();
  ProductQuantizer(const ProductQuantizer&);
  ProductQuantizer& operator=(const ProductQuantizer&);
  ProductQuantizer(ProductQuantizer&&) noexcept;
  ProductQuantizer& operator=(ProductQuantizer&&) noexcept;

  void train(const float* vectors, std::size_t n, ThreadPool* pool = nullptr,
             std::size_t iterations = 25, std::uint64_t seed = 1234);
  bool trained() const noexcept { return !centroids_.empty(); }

  std::size_t dim() const noexcept { return dim_; }
  std::size_t m() const noexcept { return m_; }
  std::size_t dsub() const noexcept { return dsub_; }
  std::size_t code_size() const noexcept { return m_; }

  void encode(const float* vector, std::uint8_t* code) const noexcept;
  void decode(const std::uint8_t* code, float* vector) const noexcept;

  /// table[j * 256 + c] = ||q_j - centroid_{j,c}||^2
  void compute_l2_table(const float* query, float* table) const noexcept;
  /// table[j * 256 + c] = <q_j, centroid_{j,c}>
  void compute_ip_table(const float* query, float* table) const noexcept;

  /// Sum of table entries selected by `code`, in order of the sub-spaces.
  float adc(const float* table, const std::uint8_t* code) const noexcept;
  /// ADC for `n` contiguous codes.
  void adc_batch(const float* table, const std::uint8_t* codes, std::size_t n,
                 float* out) const noexcept;

  /// Batched forms (no reference counterpart): codes [n][m], vectors [n][dim], tables
  /// [nq][m][256] (L2 or inner product).
  void encode_batch(const float* vectors, std::size_t n, std::uint8_t* codes) const;
  void decode_batch(const std::uint8_t* codes, std::size_t n, float* vectors) const;
  void compute_tables(const float* queries, std::size_t nq, bool inner_product, float* tables) const;

  /// m x 256 x dsub sub-centroids.
  const std::vector<float>& centroids() const noexcept { return centroids_; }
  void set_centroids(std::vector<float> centroids);

 private:
  qvh_pq* device() const;

  std::size_t dim_ = 0;
  std::size_t m_ = 0;
  std::size_t dsub_ = 0;
  std::vector<float> centroids_;
  std::shared_ptr<qvh_pq> dev_;  // the codebook on the device; immutable, shared by copies
};

}  // namespace quiver
