#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "device_util.h"
#include "quiver/quantizer.h"

namespace quiver {

namespace {

/// The reference's noexcept quantizer methods cannot fail; on the device they can, and then the
/// process stops with the message rather than returning garbage.
[[noreturn]] void fatal(const char* what, const std::exception& e) noexcept {
  std::fprintf(stderr, "quiver: %s failed: %s\n", what, e.what());
  std::abort();
}

template <class F>
void or_die(const char* what, F&& f) noexcept {
  try {
    f();
  } catch (const std::exception& e) {
    fatal(what, e);
  }
}

}  // namespace

void nearest_centroid_batch(const float* x, std::size_t n, const float* centroids, std::size_t k,
                            std::size_t dim, std::uint32_t* out) {
  if (n == 0) return;
  QUIVER_CHECK(x != nullptr && centroids != nullptr && out != nullptr, "nearest_centroid: null buffer");
  QUIVER_CHECK(k >= 1 && k <= 0xFFFFFFFFull && dim >= 1 && dim <= kMaxDimension,
               "nearest_centroid: k or dim out of range");
  internal::qvh_check(qvh_nearest_centroid(x, n, centroids, static_cast<std::uint32_t>(k),
                                           static_cast<std::uint32_t>(dim), out),
                      "nearest_centroid");
}

std::size_t nearest_centroid(const float* x, const float* centroids, std::size_t k, std::size_t dim) noexcept {
  std::uint32_t out = 0;
  if (k == 0) return 0;
  or_die("nearest_centroid", [&] { nearest_centroid_batch(x, 1, centroids, k, dim, &out); });
  return out;
}

ProductQuantizer::ProductQuantizer() = default;
ProductQuantizer::~ProductQuantizer() = default;
ProductQuantizer::ProductQuantizer(const ProductQuantizer&) = default;
ProductQuantizer& ProductQuantizer::operator=(const ProductQuantizer&) = default;
ProductQuantizer::ProductQuantizer(ProductQuantizer&&) noexcept = default;
ProductQuantizer& ProductQuantizer::operator=(ProductQuantizer&&) noexcept = default;

ProductQuantizer::ProductQuantizer(std::size_t dim, std::size_t m) : dim_(dim), m_(m) {
  QUIVER_CHECK(dim > 0 && m > 0 && dim % m == 0,
               "PQ: dimension " + std::to_string(dim) + " must be divisible by m=" + std::to_string(m));
  QUIVER_CHECK(dim <= 0xFFFFFFFFull, "PQ: dimension above 2^32 - 1");
  dsub_ = dim / m;
}

// ProductQuantizer::train of the reference (src/product_quantizer.cc:126-153): one 256-way k-means
// per sub-space over that sub-space's columns, seeded seed + j, whose assignment steps run on the
// device. The draws and sums must follow the reference's for a bit-identical codebook.
void ProductQuantizer::train(const float* vectors, std::size_t n, ThreadPool* pool, std::size_t iterations,
                             std::uint64_t seed) {
  QUIVER_CHECK(m_ > 0, "PQ is not configured");
  QUIVER_CHECK(n >= kSubCentroids, "PQ training needs at least 256 vectors, got " + std::to_string(n));
  QUIVER_CHECK(vectors != nullptr, "vectors must not be null");
  std::vector<float> book(m_ * kSubCentroids * dsub_);
  std::vector<float> columns(n * dsub_);
  for (std::size_t j = 0; j < m_; ++j) {
    const float* src = vectors + j * dsub_;
    for (std::size_t i = 0; i < n; ++i) std::memcpy(&columns[i * dsub_], src + i * dim_, dsub_ * sizeof(float));
    KMeansParams kp;
    kp.k = kSubCentroids;
    kp.iterations = iterations;
    kp.seed = seed + j;
    const std::vector<float> c = kmeans(columns.data(), n, dsub_, kp, pool);
    std::memcpy(&book[j * kSubCentroids * dsub_], c.data(), c.size() * sizeof(float));
  }
  set_centroids(std::move(book));
}

void ProductQuantizer::set_centroids(std::vector<float> centroids) {
  QUIVER_CHECK(centroids.size() == m_ * kSubCentroids * dsub_, "PQ centroid table has the wrong size");
  qvh_pq* raw = nullptr;
  internal::qvh_check(qvh_pq_create(static_cast<std::uint32_t>(dim_), static_cast<std::uint32_t>(m_),
                                    centroids.data(), &raw),
                      "ProductQuantizer");
  dev_ = std::shared_ptr<qvh_pq>(raw, qvh_pq_destroy);
  centroids_ = std::move(centroids);
}

qvh_pq* ProductQuantizer::device() const {
  QUIVER_CHECK(dev_ != nullptr, "PQ is not trained");
  return dev_.get();
}

void ProductQuantizer::encode_batch(const float* vectors, std::size_t n, std::uint8_t* codes) const {
  if (n == 0) return;
  QUIVER_CHECK(vectors != nullptr && codes != nullptr, "PQ encode: null buffer");
  internal::qvh_check(qvh_pq_encode(device(), vectors, n, codes), "PQ encode");
}

void ProductQuantizer::decode_batch(const std::uint8_t* codes, std::size_t n, float* vectors) const {
  if (n == 0) return;
  QUIVER_CHECK(codes != nullptr && vectors != nullptr, "PQ decode: null buffer");
  internal::qvh_check(qvh_pq_decode(device(), codes, n, vectors), "PQ decode");
}

void ProductQuantizer::compute_tables(const float* queries, std::size_t nq, bool inner_product, float* tables) const {
  if (nq == 0) return;
  QUIVER_CHECK(queries != nullptr && tables != nullptr, "PQ tables: null buffer");
  internal::qvh_check(qvh_pq_tables(device(), queries, nq, inner_product ? 1 : 0, tables), "PQ tables");
}

void ProductQuantizer::encode(const float* vector, std::uint8_t* code) const noexcept {
  or_die("ProductQuantizer::encode", [&] { encode_batch(vector, 1, code); });
}

void ProductQuantizer::decode(const std::uint8_t* code, float* vector) const noexcept {
  or_die("ProductQuantizer::decode", [&] { decode_batch(code, 1, vector); });
}

void ProductQuantizer::compute_l2_table(const float* query, float* table) const noexcept {
  or_die("ProductQuantizer::compute_l2_table", [&] { compute_tables(query, 1, false, table); });
}

void ProductQuantizer::compute_ip_table(const float* query, float* table) const noexcept {
  or_die("ProductQuantizer::compute_ip_table", [&] { compute_tables(query, 1, true, table); });
}

float ProductQuantizer::adc(const float* table, const std::uint8_t* code) const noexcept {
  float out = 0.0f;
  adc_batch(table, code, 1, &out);
  return out;
}

void ProductQuantizer::adc_batch(const float* table, const std::uint8_t* codes, std::size_t n,
                                 float* out) const noexcept {
  if (n == 0) return;
  or_die("ProductQuantizer::adc_batch", [&] {
    QUIVER_CHECK(table != nullptr && codes != nullptr && out != nullptr, "PQ adc: null buffer");
    internal::qvh_check(qvh_pq_adc(device(), table, codes, n, out), "PQ adc");
  });
}

}  // namespace quiver
