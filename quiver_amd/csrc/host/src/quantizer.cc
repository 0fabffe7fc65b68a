#include <cmath>
#include <cstring>
#include <limits>
#include <string>

#include "device_util.h"
#include "quiver/quantizer.h"

namespace quiver {

namespace {

constexpr std::size_t kBook = ProductQuantizer::kSubCentroids;

/// out[c] = sum over t of (x_t - book[c][t])^2 for the 256 codewords of one sub-space, each sum
/// taken in order of t from 0.0f with separately rounded products: CentroidTable::l2
/// (src/internal/centroid_table.h:65-75) visits t in the outer loop, which gives every c the same
/// sequence of additions.
void codeword_l2(const float* x, const float* book, std::size_t dsub, float* out) noexcept {
  for (std::size_t c = 0; c < kBook; ++c) {
    const float* w = book + c * dsub;
    float acc = 0.0f;
    for (std::size_t t = 0; t < dsub; ++t) {
      const float diff = x[t] - w[t];
      acc += diff * diff;
    }
    out[c] = acc;
  }
}

/// out[c] = sum over t of x_t * book[c][t], in order of t from 0.0f (CentroidTable::dot,
/// src/internal/centroid_table.h:78-85).
void codeword_dot(const float* x, const float* book, std::size_t dsub, float* out) noexcept {
  for (std::size_t c = 0; c < kBook; ++c) {
    const float* w = book + c * dsub;
    float acc = 0.0f;
    for (std::size_t t = 0; t < dsub; ++t) acc += x[t] * w[t];
    out[c] = acc;
  }
}

/// The index CentroidTable::argmin_n returns (src/internal/centroid_table.h:155-170): the smallest
/// value that is not NaN (+inf if every value is NaN), then the first index holding a value equal
/// to it; 0 when none does (all NaN). Signed zeros compare equal, so which zero the minimum holds
/// does not matter.
std::size_t first_minimum(const float* v, std::size_t n) noexcept {
  float lowest = std::numeric_limits<float>::infinity();
  for (std::size_t i = 0; i < n; ++i) {
    if (v[i] < lowest) lowest = v[i];
  }
  for (std::size_t i = 0; i < n; ++i) {
    if (v[i] == lowest) return i;
  }
  return 0;
}

/// simd::l2sqr with the AVX2 kernels (src/simd/kernels_avx2.cc:35-56), the kernel the reference
/// dispatches to on x86-64 (src/simd/dispatch.cc:108-117): eight-lane fused accumulators over
/// blocks of 32 elements and then of 8, the pairwise horizontal sum, and the tail as GCC compiles
/// it (the first four remaining products rounded and added, the rest fused).
float l2sqr_avx2_order(const float* a, const float* b, std::size_t dim) noexcept {
  float acc[4][8] = {};
  std::size_t i = 0;
  for (; i + 32 <= dim; i += 32) {
    for (std::size_t block = 0; block < 4; ++block) {
      for (std::size_t lane = 0; lane < 8; ++lane) {
        const float diff = a[i + block * 8 + lane] - b[i + block * 8 + lane];
        acc[block][lane] = std::fma(diff, diff, acc[block][lane]);
      }
    }
  }
  for (; i + 8 <= dim; i += 8) {
    for (std::size_t lane = 0; lane < 8; ++lane) {
      const float diff = a[i + lane] - b[i + lane];
      acc[0][lane] = std::fma(diff, diff, acc[0][lane]);
    }
  }
  float lanes[8];
  for (std::size_t lane = 0; lane < 8; ++lane) {
    lanes[lane] = (acc[0][lane] + acc[1][lane]) + (acc[2][lane] + acc[3][lane]);
  }
  float half[4];
  for (std::size_t j = 0; j < 4; ++j) half[j] = lanes[j] + lanes[j + 4];
  float sum = (half[0] + half[1]) + (half[2] + half[3]);
  const std::size_t rounded_end = i + (dim - i) / 4 * 4;
  for (; i < rounded_end; ++i) {
    const float diff = a[i] - b[i];
    sum += diff * diff;
  }
  for (; i < dim; ++i) {
    const float diff = a[i] - b[i];
    sum = std::fma(diff, diff, sum);
  }
  return sum;
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

// nearest_centroid (src/product_quantizer.cc:14-27) for one point, on the host: the AVX2-order
// distance to each centroid in turn, a strictly smaller one replacing the best. It cannot fail,
// like the reference's; nearest_centroid_batch runs the same arithmetic on the device.
std::size_t nearest_centroid(const float* x, const float* centroids, std::size_t k, std::size_t dim) noexcept {
  std::size_t best = 0;
  float best_dist = std::numeric_limits<float>::infinity();
  for (std::size_t c = 0; c < k; ++c) {
    const float dist = l2sqr_avx2_order(x, centroids + c * dim, dim);
    if (dist < best_dist) {
      best_dist = dist;
      best = c;
    }
  }
  return best;
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

// The per-vector methods below run on the host, in the reference's float order, so they are
// bit-identical to it and to the device batch methods, and they cannot fail (the reference's are
// noexcept). Before a codebook is installed they leave their outputs untouched (encode, decode,
// tables) or return 0 (adc).

void ProductQuantizer::encode(const float* vector, std::uint8_t* code) const noexcept {
  if (!trained()) return;
  float dist[kBook];
  for (std::size_t j = 0; j < m_; ++j) {
    codeword_l2(vector + j * dsub_, centroids_.data() + j * kBook * dsub_, dsub_, dist);
    code[j] = static_cast<std::uint8_t>(first_minimum(dist, kBook));
  }
}

void ProductQuantizer::decode(const std::uint8_t* code, float* vector) const noexcept {
  if (!trained()) return;
  for (std::size_t j = 0; j < m_; ++j) {
    const float* word = centroids_.data() + (j * kBook + code[j]) * dsub_;
    std::memcpy(vector + j * dsub_, word, dsub_ * sizeof(float));
  }
}

void ProductQuantizer::compute_l2_table(const float* query, float* table) const noexcept {
  if (!trained()) return;
  for (std::size_t j = 0; j < m_; ++j) {
    codeword_l2(query + j * dsub_, centroids_.data() + j * kBook * dsub_, dsub_, table + j * kBook);
  }
}

void ProductQuantizer::compute_ip_table(const float* query, float* table) const noexcept {
  if (!trained()) return;
  for (std::size_t j = 0; j < m_; ++j) {
    codeword_dot(query + j * dsub_, centroids_.data() + j * kBook * dsub_, dsub_, table + j * kBook);
  }
}

// ProductQuantizer::adc (src/product_quantizer.cc:188-192): the table entries a code selects,
// added in order of the sub-spaces from 0.0f.
float ProductQuantizer::adc(const float* table, const std::uint8_t* code) const noexcept {
  float sum = 0.0f;
  for (std::size_t j = 0; j < m_; ++j) sum += table[j * kBook + code[j]];
  return sum;
}

// ProductQuantizer::adc_batch (src/product_quantizer.cc:194-217) interleaves four codes, but each
// code's sum is still taken in order of j, so every out[i] equals adc of code i.
void ProductQuantizer::adc_batch(const float* table, const std::uint8_t* codes, std::size_t n,
                                 float* out) const noexcept {
  for (std::size_t i = 0; i < n; ++i) out[i] = adc(table, codes + i * m_);
}

}  // namespace quiver
