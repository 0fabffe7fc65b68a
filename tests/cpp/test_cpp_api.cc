// The public C++ API (quiver/flat_index.h, quiver/ivfpq_index.h, quiver/quantizer.h) driven the way
// a C++ caller of the reference drives it: the behaviours its tests check for the flat and IVF-PQ
// indexes, k-means, nearest_centroid and the product quantizer (tests/test_flat.cc,
// tests/test_quantizer.cc, tests/test_regressions.cc), compiled against this package's headers and
// run on the GPU. Prints one line per case and exits non-zero on a failure.

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <cstring>
#include <functional>
#include <limits>
#include <random>
#include <string>
#include <thread>
#include <unordered_set>
#include <vector>

#include "qvh.h"
#include "quiver/common.h"
#include "quiver/filter.h"
#include "quiver/flat_index.h"
#include "quiver/ivfpq_index.h"
#include "quiver/quantizer.h"

namespace {

int g_failures = 0;

#define EXPECT(cond)                                                           \
  do {                                                                         \
    if (!(cond)) {                                                             \
      std::printf("    expectation failed: %s (line %d)\n", #cond, __LINE__); \
      ++g_failures;                                                            \
    }                                                                          \
  } while (0)

template <class F>
bool throws_error(F&& f) {
  try {
    f();
  } catch (const quiver::Error&) {
    return true;
  }
  return false;
}

std::vector<float> normal_vectors(std::size_t n, std::size_t dim, std::uint64_t seed) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> unit(0.0f, 1.0f);
  std::vector<float> v(n * dim);
  for (float& x : v) x = unit(rng);
  return v;
}

std::vector<float> blob_vectors(std::size_t n, std::size_t dim, std::size_t clusters, std::uint64_t seed) {
  std::mt19937_64 crng(4242 + clusters), rng(seed);
  std::normal_distribution<float> unit(0.0f, 1.0f);
  std::vector<float> centers(clusters * dim);
  for (float& x : centers) x = 3.0f * unit(crng);
  std::uniform_int_distribution<std::size_t> pick(0, clusters - 1);
  std::vector<float> v(n * dim);
  for (std::size_t i = 0; i < n; ++i) {
    const std::size_t c = pick(rng);
    for (std::size_t j = 0; j < dim; ++j) v[i * dim + j] = centers[c * dim + j] + unit(rng);
  }
  return v;
}

// The k nearest rows by squared L2 distance in double precision.
std::vector<std::size_t> brute_force(const std::vector<float>& base, const float* q, std::size_t dim,
                                     std::size_t k) {
  const std::size_t n = base.size() / dim;
  std::vector<std::pair<double, std::size_t>> d(n);
  for (std::size_t i = 0; i < n; ++i) {
    double s = 0;
    for (std::size_t j = 0; j < dim; ++j) {
      const double t = static_cast<double>(q[j]) - base[i * dim + j];
      s += t * t;
    }
    d[i] = {s, i};
  }
  std::partial_sort(d.begin(), d.begin() + static_cast<std::ptrdiff_t>(k), d.end());
  std::vector<std::size_t> out(k);
  for (std::size_t i = 0; i < k; ++i) out[i] = d[i].second;
  return out;
}

double recall(const std::vector<std::size_t>& truth, const std::vector<quiver::Neighbor>& got) {
  std::unordered_set<std::size_t> t(truth.begin(), truth.end());
  std::size_t hit = 0;
  for (const auto& nb : got) hit += t.count(static_cast<std::size_t>(nb.label));
  return static_cast<double>(hit) / static_cast<double>(truth.size());
}

void flat_matches_brute_force() {
  const std::size_t dim = 16, n = 2000, k = 10;
  const auto base = normal_vectors(n, dim, 1);
  const auto queries = normal_vectors(20, dim, 2);
  quiver::FlatIndex index(dim);
  index.add(base.data(), n);
  EXPECT(index.size() == n);
  for (std::size_t i = 0; i < 20; ++i) {
    const auto r = index.search(queries.data() + i * dim, k);
    EXPECT(r.size() == k);
    const auto truth = brute_force(base, queries.data() + i * dim, dim, k);
    for (std::size_t j = 0; j < k && j < r.size(); ++j) EXPECT(r[j].label == truth[j]);
    EXPECT(std::is_sorted(r.begin(), r.end()));
  }
  // The batched call returns the same rows.
  std::vector<quiver::Label> labels(20 * k);
  std::vector<float> dist(20 * k);
  index.search_batch(queries.data(), 20, k, labels.data(), dist.data());
  for (std::size_t i = 0; i < 20; ++i) {
    const auto r = index.search(queries.data() + i * dim, k);
    for (std::size_t j = 0; j < k; ++j) EXPECT(labels[i * k + j] == r[j].label && dist[i * k + j] == r[j].distance);
  }
}

void flat_cosine_and_inner_product() {
  const std::size_t dim = 8, n = 500;
  auto base = normal_vectors(n, dim, 3);
  for (const auto metric : {quiver::Metric::kCosine, quiver::Metric::kInnerProduct}) {
    quiver::FlatIndex index(dim, metric);
    index.add(base.data(), n);
    std::vector<float> q(base.begin() + 7 * dim, base.begin() + 8 * dim);
    if (metric == quiver::Metric::kCosine) {
      for (float& x : q) x *= 3.0f;  // the same direction: distance 0 to row 7
      const auto r = index.search(q.data(), 1);
      EXPECT(r.size() == 1 && r[0].label == 7 && std::fabs(r[0].distance) < 1e-5f);
    } else {
      const auto r = index.search(q.data(), 5);
      EXPECT(r.size() == 5 && std::is_sorted(r.begin(), r.end()));
    }
  }
}

void flat_fewer_than_k_and_filters() {
  const std::size_t dim = 4;
  const auto base = normal_vectors(5, dim, 4);
  quiver::FlatIndex index(dim);
  const quiver::Label labels[5] = {10, 11, 12, 13, 14};
  index.add(base.data(), 5, labels);
  EXPECT(index.search(base.data(), 10).size() == 5);
  const quiver::LabelSetFilter only{11, 13};
  const auto r = index.search(base.data(), 10, &only);
  EXPECT(r.size() == 2);
  for (const auto& nb : r) EXPECT(nb.label == 11 || nb.label == 13);
  std::vector<quiver::Label> out(10);
  std::vector<float> dist(10);
  index.search_batch(base.data(), 1, 10, out.data(), dist.data(), &only);
  EXPECT(out[2] == quiver::kInvalidLabel && std::isinf(dist[2]));
  const quiver::Label sentinel = quiver::kInvalidLabel;
  EXPECT(throws_error([&] { index.add(base.data(), 1, &sentinel); }));
  std::vector<float> bad(dim, 1.0f);
  bad[1] = std::nanf("");
  EXPECT(throws_error([&] { index.add(bad.data(), 1); }));
}

void flat_save_load(const std::string& dir) {
  const std::size_t dim = 12, n = 300;
  const auto base = normal_vectors(n, dim, 5);
  quiver::FlatIndex index(dim, quiver::Metric::kCosine);
  index.add(base.data(), n);
  const std::string path = dir + "/flat.qvr";
  index.save(path);
  const auto loaded = quiver::FlatIndex::load(path);
  EXPECT(loaded.size() == n && loaded.dim() == dim && loaded.metric() == quiver::Metric::kCosine);
  for (std::size_t i = 0; i < 10; ++i) {
    const auto a = index.search(base.data() + i * dim, 5), b = loaded.search(base.data() + i * dim, 5);
    EXPECT(a.size() == b.size());
    for (std::size_t j = 0; j < a.size() && j < b.size(); ++j) EXPECT(a[j].label == b[j].label && a[j].distance == b[j].distance);
  }
}

void ivfpq_recall_save_load_and_errors(const std::string& dir) {
  const std::size_t dim = 32, n = 6000, nq = 50, k = 10;
  const auto base = blob_vectors(n, dim, 40, 6);
  const auto queries = blob_vectors(nq, dim, 40, 7);
  quiver::IvfPqParams p;
  p.dim = dim;
  p.nlist = 64;
  p.m = 16;
  p.store_vectors = true;
  quiver::IvfPqIndex index(p);
  EXPECT(!index.is_trained());
  EXPECT(throws_error([&] { index.add(base.data(), n); }));  // must train first
  index.train(base.data(), n);
  EXPECT(index.is_trained());
  EXPECT(throws_error([&] { index.train(base.data(), n); }));  // once only
  index.add(base.data(), n);
  EXPECT(index.size() == n);
  quiver::IvfPqSearchParams sp;
  sp.nprobe = 16;
  sp.refine_factor = 4;
  double total = 0;
  for (std::size_t i = 0; i < nq; ++i) {
    const auto r = index.search(queries.data() + i * dim, k, sp);
    EXPECT(r.size() == k && std::is_sorted(r.begin(), r.end()));
    total += recall(brute_force(base, queries.data() + i * dim, dim, k), r);
  }
  std::printf("    recall@10 (nprobe 16, refine 4): %.3f\n", total / nq);
  EXPECT(total / nq >= 0.9);
  // Refine over everything (k * refine_factor saturates at the count) with every list probed is exact.
  sp.nprobe = p.nlist;
  sp.refine_factor = std::size_t{1} << 63;
  for (std::size_t i = 0; i < 5; ++i) {
    const auto r = index.search(queries.data() + i * dim, 2, sp);
    const auto truth = brute_force(base, queries.data() + i * dim, dim, 2);
    EXPECT(r.size() == 2 && r[0].label == truth[0]);
  }
  // A filter admits only its labels.
  const quiver::LabelSetFilter even = [&] {
    quiver::LabelSetFilter f;
    for (quiver::Label l = 0; l < n; l += 2) f.insert(l);
    return f;
  }();
  sp.nprobe = 16;
  sp.refine_factor = 0;
  sp.filter = &even;
  for (const auto& nb : index.search(queries.data(), k, sp)) EXPECT(nb.label % 2 == 0);
  sp.filter = nullptr;
  const std::string path = dir + "/ivf.qvr";
  index.save(path);
  const auto loaded = quiver::IvfPqIndex::load(path);
  EXPECT(loaded.size() == n && loaded.is_trained());
  for (std::size_t i = 0; i < 10; ++i) {
    const auto a = index.search(queries.data() + i * dim, 5, sp), b = loaded.search(queries.data() + i * dim, 5, sp);
    EXPECT(a.size() == b.size());
    for (std::size_t j = 0; j < a.size() && j < b.size(); ++j) EXPECT(a[j].label == b[j].label && a[j].distance == b[j].distance);
  }
}

double l2_double(const float* a, const float* b, std::size_t dim) {
  double s = 0;
  for (std::size_t j = 0; j < dim; ++j) {
    const double t = static_cast<double>(a[j]) - b[j];
    s += t * t;
  }
  return s;
}

double dot_double(const float* a, const float* b, std::size_t dim) {
  double s = 0;
  for (std::size_t j = 0; j < dim; ++j) s += static_cast<double>(a[j]) * b[j];
  return s;
}

// tests/test_quantizer.cc:20-37: three well separated clusters; nearest_centroid finds each centre's
// centroid within 0.05.
void kmeans_recovers_separated_clusters() {
  const std::size_t dim = 4, per = 200, k = 3;
  const float centers[3][4] = {{0, 0, 0, 0}, {10, 10, 0, 0}, {0, 0, 10, 10}};
  const auto noise = normal_vectors(per * k, dim, 1);
  std::vector<float> data;
  for (std::size_t c = 0; c < k; ++c)
    for (std::size_t i = 0; i < per; ++i)
      for (std::size_t j = 0; j < dim; ++j) data.push_back(centers[c][j] + 0.1f * noise[(c * per + i) * dim + j]);
  quiver::KMeansParams kp;
  kp.k = k;
  const auto cent = quiver::kmeans(data.data(), per * k, dim, kp);
  for (const auto& c : centers) {
    const std::size_t nearest = quiver::nearest_centroid(c, cent.data(), k, dim);
    EXPECT(nearest < k && l2_double(c, cent.data() + nearest * dim, dim) < 0.05);
  }
  // The first of equal centroids wins; no finite distance: index 0.
  const std::vector<float> twins = {5, 5, 1, 1, 1, 1};
  const float origin[2] = {1, 1};
  EXPECT(quiver::nearest_centroid(origin, twins.data(), 3, 2) == 1);
  const std::vector<float> huge = {3e38f, 3e38f, -3e38f, -3e38f};
  EXPECT(quiver::nearest_centroid(origin, huge.data(), 2, 2) == 0);
}

// tests/test_quantizer.cc:39-48: identical points force empty clusters; no NaN comes out.
void kmeans_handles_duplicate_points() {
  std::vector<float> data(1000 * 2, 1.0f);
  for (std::size_t i = 0; i < 20; ++i) data[i * 2] = static_cast<float>(i);
  quiver::KMeansParams kp;
  kp.k = 16;
  for (float x : quiver::kmeans(data.data(), 1000, 2, kp)) EXPECT(std::isfinite(x));
}

// tests/test_quantizer.cc:50-68: more sub-quantizers reconstruct better.
void pq_reconstruction_beats_coarser_codes() {
  const std::size_t dim = 32, n = 4000;
  const auto data = blob_vectors(n, dim, 10, 3);
  double prev = 1e30;
  for (std::size_t m : {4u, 8u, 16u}) {
    quiver::ProductQuantizer pq(dim, m);
    pq.train(data.data(), n);
    EXPECT(pq.trained() && pq.code_size() == m && pq.dsub() == dim / m);
    std::vector<std::uint8_t> codes(n * m);
    std::vector<float> back(n * dim);
    pq.encode_batch(data.data(), n, codes.data());
    pq.decode_batch(codes.data(), n, back.data());
    std::vector<std::uint8_t> one(m);
    std::vector<float> rec(dim);
    for (std::size_t i = 0; i < n; i += 397) {  // the per-vector calls agree with the batch
      pq.encode(data.data() + i * dim, one.data());
      EXPECT(std::equal(one.begin(), one.end(), codes.begin() + static_cast<std::ptrdiff_t>(i * m)));
      pq.decode(one.data(), rec.data());
      EXPECT(std::equal(rec.begin(), rec.end(), back.begin() + static_cast<std::ptrdiff_t>(i * dim)));
    }
    double err = 0;
    for (std::size_t i = 0; i < n * dim; ++i) err += (data[i] - back[i]) * static_cast<double>(data[i] - back[i]);
    err /= static_cast<double>(n * dim);
    std::printf("    m=%zu reconstruction mse %.4f\n", m, err);
    EXPECT(err < prev);
    prev = err;
  }
  EXPECT(prev < 0.3);
}

// tests/test_quantizer.cc:70-92: ADC over the L2 table is the distance to the reconstruction, and
// over the IP table the inner product with it; adc_batch equals adc.
void pq_adc_equals_distance_to_reconstruction() {
  const std::size_t dim = 16, n = 1000, m = 4;
  const auto data = normal_vectors(n, dim, 4);
  quiver::ProductQuantizer pq(dim, m);
  pq.train(data.data(), n);
  const auto q = normal_vectors(1, dim, 5);
  std::vector<float> l2t(m * 256), ipt(m * 256);
  pq.compute_l2_table(q.data(), l2t.data());
  pq.compute_ip_table(q.data(), ipt.data());
  std::vector<std::uint8_t> codes(7 * m);
  for (std::size_t i = 0; i < 7; ++i) pq.encode(data.data() + i * dim, codes.data() + i * m);
  std::vector<float> batch(7);
  pq.adc_batch(l2t.data(), codes.data(), 7, batch.data());
  for (std::size_t i = 0; i < 7; ++i) {
    std::vector<float> rec(dim);
    pq.decode(codes.data() + i * m, rec.data());
    const float a = pq.adc(l2t.data(), codes.data() + i * m);
    EXPECT(std::fabs(a - l2_double(q.data(), rec.data(), dim)) < 1e-3);
    EXPECT(batch[i] == a);
    EXPECT(std::fabs(pq.adc(ipt.data(), codes.data() + i * m) - dot_double(q.data(), rec.data(), dim)) < 1e-3);
  }
  // A copy shares the trained codebook; set_centroids installs one directly.
  const quiver::ProductQuantizer copy = pq;
  quiver::ProductQuantizer other(dim, m);
  other.set_centroids(pq.centroids());
  std::vector<std::uint8_t> c1(m), c2(m);
  copy.encode(data.data() + 3 * dim, c1.data());
  other.encode(data.data() + 3 * dim, c2.data());
  EXPECT(std::equal(c1.begin(), c1.end(), codes.begin() + 3 * static_cast<std::ptrdiff_t>(m)) && c1 == c2);
}

bool same_bits(const float* a, const float* b, std::size_t n) { return std::memcmp(a, b, n * sizeof(float)) == 0; }

/// Bit-identical, except that two NaNs match whatever their sign: a NaN codeword gives the host
/// (x86, like the reference) a positive NaN table entry and the device a negative one. A NaN
/// distance never ranks (the scans map it to +inf), so only the table's bits can show the sign.
bool same_bits_or_nan(const float* a, const float* b, std::size_t n) {
  for (std::size_t i = 0; i < n; ++i) {
    if (std::isnan(a[i]) && std::isnan(b[i])) continue;
    if (std::memcmp(a + i, b + i, sizeof(float)) != 0) return false;
  }
  return true;
}

// The per-vector ProductQuantizer methods and nearest_centroid run on the host, the *_batch methods
// and the C-ABI's qvh_pq_adc on the device (those are checked against the reference's golden
// vectors and the oracle in tests/test_pq_gpu.py). Both follow the reference's float order
// (src/product_quantizer.cc:14-27,165-217, src/internal/centroid_table.h:65-85,155-170), so they
// must agree bit for bit: sub-spaces of 1 to 8 dims, NaN and infinite codewords (argmin_n takes
// the first index holding the smallest non-NaN value, 0 when all are NaN), and point dims 1-70,
// which cover every tail length of the AVX2-order distance.
void pq_per_vector_host_matches_device_batch() {
  const std::pair<std::size_t, std::size_t> shapes[] = {{128, 32}, {100, 25}, {96, 12}, {30, 30}, {56, 7}};
  for (const auto& [dim, m] : shapes) {
    const std::size_t dsub = dim / m, n = 300;
    auto book = normal_vectors(m * 256 * dsub, 1, dim + m);
    // sub-space 0: codeword 0 NaN, 1-255 +inf (the first +inf wins); sub-space 1: every codeword NaN
    const float nan = std::numeric_limits<float>::quiet_NaN(), inf = std::numeric_limits<float>::infinity();
    for (std::size_t c = 0; c < 256; ++c) {
      for (std::size_t t = 0; t < dsub; ++t) {
        book[c * dsub + t] = c == 0 ? nan : inf;
        book[(256 + c) * dsub + t] = nan;
      }
    }
    quiver::ProductQuantizer pq(dim, m);
    pq.set_centroids(book);
    const auto x = normal_vectors(n, dim, 77 + dim);
    std::vector<std::uint8_t> batch(n * m), one(m);
    pq.encode_batch(x.data(), n, batch.data());
    std::size_t code_mismatch = 0;
    for (std::size_t i = 0; i < n; ++i) {
      pq.encode(x.data() + i * dim, one.data());
      code_mismatch += !std::equal(one.begin(), one.end(), batch.begin() + static_cast<std::ptrdiff_t>(i * m));
    }
    EXPECT(code_mismatch == 0);
    EXPECT(batch[0] == 1 && batch[1] == 0);
    std::vector<float> dec(n * dim), rec(dim);
    pq.decode_batch(batch.data(), n, dec.data());
    for (std::size_t i = 0; i < n; i += 7) {
      pq.decode(batch.data() + i * m, rec.data());
      EXPECT(same_bits(rec.data(), dec.data() + i * dim, dim));
    }
    const std::size_t nq = 5;
    std::vector<float> l2(nq * m * 256), ip(nq * m * 256), t(m * 256);
    pq.compute_tables(x.data(), nq, false, l2.data());
    pq.compute_tables(x.data(), nq, true, ip.data());
    for (std::size_t q = 0; q < nq; ++q) {
      pq.compute_l2_table(x.data() + q * dim, t.data());
      EXPECT(same_bits_or_nan(t.data(), l2.data() + q * m * 256, m * 256));
      pq.compute_ip_table(x.data() + q * dim, t.data());
      EXPECT(same_bits_or_nan(t.data(), ip.data() + q * m * 256, m * 256));
    }
    // adc over the inner-product table of query 0 (finite entries only in sub-spaces >= 2)
    qvh_pq* dev = nullptr;
    EXPECT(qvh_pq_create(static_cast<std::uint32_t>(dim), static_cast<std::uint32_t>(m), book.data(), &dev) == QVH_OK);
    std::vector<float> host_adc(n), dev_adc(n), single(n);
    pq.adc_batch(ip.data(), batch.data(), n, host_adc.data());
    EXPECT(qvh_pq_adc(dev, ip.data(), batch.data(), n, dev_adc.data()) == QVH_OK);
    for (std::size_t i = 0; i < n; ++i) single[i] = pq.adc(ip.data(), batch.data() + i * m);
    qvh_pq_destroy(dev);
    EXPECT(same_bits_or_nan(host_adc.data(), dev_adc.data(), n) && same_bits_or_nan(single.data(), dev_adc.data(), n));
  }
  for (std::size_t dim = 1; dim <= 70; ++dim) {
    const std::size_t k = 97, n = 40;
    auto cent = normal_vectors(k, dim, 1000 + dim);
    for (std::size_t j = 0; j < dim; ++j) cent[5 * dim + j] = cent[60 * dim + j];  // equal centroids
    const auto x = normal_vectors(n, dim, 2000 + dim);
    std::vector<std::uint32_t> batch(n);
    quiver::nearest_centroid_batch(x.data(), n, cent.data(), k, dim, batch.data());
    std::size_t mismatch = 0;
    for (std::size_t i = 0; i < n; ++i) {
      mismatch += quiver::nearest_centroid(x.data() + i * dim, cent.data(), k, dim) != batch[i];
    }
    EXPECT(mismatch == 0);
    // a point on the duplicated centroid picks the first copy
    EXPECT(quiver::nearest_centroid(cent.data() + 60 * dim, cent.data(), k, dim) == 5);
  }
}

// tests/test_quantizer.cc:94-99
void pq_rejects_bad_shapes() {
  EXPECT(throws_error([] { quiver::ProductQuantizer(10, 3); }));
  quiver::ProductQuantizer pq(8, 2);
  const auto few = normal_vectors(100, 8, 1);
  EXPECT(throws_error([&] { pq.train(few.data(), 100); }));
  EXPECT(throws_error([&] { pq.set_centroids(std::vector<float>(7)); }));
  EXPECT(throws_error([&] { quiver::ProductQuantizer().train(few.data(), 100); }));
}

// src/ivfpq_index.cc:218-249: add() encodes without holding the index lock and takes the exclusive
// lock only to append, so search_batch calls from another thread keep returning while a 1M-vector
// add() encodes. Each of them sees the index as it was before the add or as it is after it, never
// a partial state, and the add's lists equal those of the same add without concurrent searches.
void ivfpq_search_proceeds_during_add() {
  using clock = std::chrono::steady_clock;
  const std::size_t dim = 128, n0 = 20000, nbig = 1000000, nq = 64, k = 10;
  const auto train = blob_vectors(n0, dim, 50, 11);
  const auto big = blob_vectors(nbig, dim, 50, 12);
  const auto q = blob_vectors(nq, dim, 50, 13);
  quiver::IvfPqParams p;
  p.dim = dim;
  p.nlist = 1024;
  p.m = 32;
  quiver::IvfPqIndex index(p), serial(p);
  index.train(train.data(), n0);
  serial.set_trained(index.centroids().data(), index.codebook().data());
  index.add(train.data(), n0);
  serial.add(train.data(), n0);
  quiver::IvfPqSearchParams sp;
  sp.nprobe = 8;
  auto search = [&](quiver::IvfPqIndex& ix) {
    std::pair<std::vector<quiver::Label>, std::vector<float>> r{std::vector<quiver::Label>(nq * k),
                                                                std::vector<float>(nq * k)};
    ix.search_batch(q.data(), nq, k, r.first.data(), r.second.data(), sp);
    return r;
  };
  const auto before = search(index);
  std::atomic<bool> started{false}, finished{false};
  clock::time_point add_begin, add_end;
  std::thread adder([&] {
    add_begin = clock::now();
    started = true;
    index.add(big.data(), nbig);
    add_end = clock::now();
    finished = true;
  });
  while (!started) std::this_thread::yield();
  std::vector<std::pair<clock::time_point, decltype(search(index))>> done;
  while (!finished) {
    auto r = search(index);
    done.emplace_back(clock::now(), std::move(r));
  }
  adder.join();
  serial.add(big.data(), nbig);
  const auto after = search(index);
  EXPECT(after == search(serial));
  EXPECT(index.list_labels() == serial.list_labels() && index.list_codes() == serial.list_codes());
  std::size_t during = 0, mixed = 0;
  double max_gap = 0;
  auto last = add_begin;
  for (const auto& [t, r] : done) {
    if (t >= add_end) break;
    ++during;
    mixed += !(r == before || r == after);
    max_gap = std::max(max_gap, std::chrono::duration<double>(t - last).count());
    last = t;
  }
  max_gap = std::max(max_gap, std::chrono::duration<double>(add_end - last).count());
  const double add_s = std::chrono::duration<double>(add_end - add_begin).count();
  std::printf("    add of %zu vectors %.1f ms; %zu searches returned during it; longest wait between them "
              "%.1f ms\n", nbig, add_s * 1e3, during, max_gap * 1e3);
  EXPECT(mixed == 0);
  EXPECT(during >= 5);
  // Holding the exclusive lock across the encode would stall every search for most of the add.
  EXPECT(max_gap < 0.35 * add_s);
}

// IvfPqIndex::list_sizes / memory_bytes (src/ivfpq_index.cc:446-463): the sizes add up to size(),
// and the byte count follows the reference's accounting.
void ivfpq_list_sizes_and_memory_bytes() {
  const std::size_t dim = 16, n = 3000;
  const auto base = blob_vectors(n, dim, 20, 8);
  for (const bool store : {false, true}) {
    quiver::IvfPqParams p;
    p.dim = dim;
    p.nlist = 32;
    p.m = 8;
    p.store_vectors = store;
    quiver::IvfPqIndex index(p);
    EXPECT(index.list_sizes().size() == p.nlist);
    index.train(base.data(), n);
    index.add(base.data(), n);
    const auto sizes = index.list_sizes();
    std::size_t total = 0;
    for (std::size_t s : sizes) total += s;
    EXPECT(total == n);
    const std::size_t expect = (p.nlist * dim + p.m * 256 * (dim / p.m) + p.nlist * p.m * 256) * sizeof(float) +
                               n * p.m + n * sizeof(quiver::Label) + (store ? n * dim * sizeof(float) : 0);
    EXPECT(index.memory_bytes() == expect);
  }
}

}  // namespace

int main() {
  const std::string dir = (std::filesystem::temp_directory_path() / ("quiver_cpp_api_" + std::to_string(::getpid()))).string();
  std::filesystem::create_directories(dir);
  const std::pair<const char*, std::function<void()>> cases[] = {
      {"flat_matches_brute_force", flat_matches_brute_force},
      {"flat_cosine_and_inner_product", flat_cosine_and_inner_product},
      {"flat_fewer_than_k_and_filters", flat_fewer_than_k_and_filters},
      {"flat_save_load", [&] { flat_save_load(dir); }},
      {"ivfpq_recall_save_load_and_errors", [&] { ivfpq_recall_save_load_and_errors(dir); }},
      {"kmeans_recovers_separated_clusters", kmeans_recovers_separated_clusters},
      {"kmeans_handles_duplicate_points", kmeans_handles_duplicate_points},
      {"pq_reconstruction_beats_coarser_codes", pq_reconstruction_beats_coarser_codes},
      {"pq_adc_equals_distance_to_reconstruction", pq_adc_equals_distance_to_reconstruction},
      {"pq_per_vector_host_matches_device_batch", pq_per_vector_host_matches_device_batch},
      {"pq_rejects_bad_shapes", pq_rejects_bad_shapes},
      {"ivfpq_list_sizes_and_memory_bytes", ivfpq_list_sizes_and_memory_bytes},
      {"ivfpq_search_proceeds_during_add", ivfpq_search_proceeds_during_add},
  };
  for (const auto& [name, fn] : cases) {
    const int before = g_failures;
    std::printf("case %s\n", name);
    std::fflush(stdout);
    try {
      fn();
    } catch (const std::exception& e) {
      std::printf("    unexpected exception: %s\n", e.what());
      ++g_failures;
    }
    std::printf("  %s\n", g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
  }
  std::filesystem::remove_all(dir);
  std::printf("%s\n", g_failures == 0 ? "all cases passed" : "failures");
  return g_failures == 0 ? 0 : 1;
}
