// C-ABI shim over the compiled reference library (TheWiseGhost/quiver), used ONLY as a checker:
// it produces the golden fixtures under tests/golden/ and times the reference CPU path for the
// bench's cpu_baseline. Built by oracle/Makefile into oracle/_ref/ together with the reference's
// own sources, compiled where they lie; nothing here is part of the product.
//
// Each entry point wraps one public reference call:
//   FlatIndex::add / search_batch          include/quiver/flat_index.h:27-36
//   IvfPqIndex::train / add / search_batch include/quiver/ivfpq_index.h:53-64
//   IvfPqIndex::save / load                include/quiver/ivfpq_index.h:66-67
//   kmeans                                 include/quiver/quantizer.h:57-58
//   ProductQuantizer::encode / tables      include/quiver/quantizer.h:90-104
//   simd::normalize / active().l2sqr,dot   include/quiver/distance.h:28-47
// Filters are built the way the Python binding builds them (python/quiver_ext.cc:40-51).
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "quiver/distance.h"
#include "quiver/filter.h"
#include "quiver/flat_index.h"
#include "quiver/ivfpq_index.h"
#include "quiver/quantizer.h"
#include "quiver/thread_pool.h"

namespace {

thread_local std::string g_err;

quiver::ThreadPool* pool_for(std::size_t threads) {
  if (threads == 0) return &quiver::ThreadPool::global();
  static std::mutex mu;
  static std::map<std::size_t, std::unique_ptr<quiver::ThreadPool>> pools;
  std::lock_guard lock(mu);
  auto& p = pools[threads];
  if (!p) p = std::make_unique<quiver::ThreadPool>(threads);
  return p.get();
}

std::unique_ptr<quiver::Filter> make_filter(const std::uint64_t* p, std::int64_t n) {
  if (n < 0) return nullptr;
  const auto count = static_cast<std::size_t>(n);
  const std::uint64_t max_label = count == 0 ? 0 : *std::max_element(p, p + count);
  if (max_label < (std::uint64_t{1} << 32) && max_label / 64 <= 16 * count + 1024) {
    auto f = std::make_unique<quiver::BitsetFilter>(static_cast<std::size_t>(max_label) + 1);
    for (std::size_t i = 0; i < count; ++i) f->insert(p[i]);
    return f;
  }
  return std::make_unique<quiver::LabelSetFilter>(p, p + count);
}

template <class F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

}  // namespace

extern "C" {

const char* qref_last_error(void) { return g_err.c_str(); }

const char* qref_simd_isa(void) {
  static std::string s(quiver::simd::to_string(quiver::simd::active().isa));
  return s.c_str();
}

float qref_l2sqr(const float* a, const float* b, std::size_t dim) {
  return quiver::simd::active().l2sqr(a, b, dim);
}
float qref_dot(const float* a, const float* b, std::size_t dim) {
  return quiver::simd::active().dot(a, b, dim);
}
void qref_normalize(float* v, std::size_t n, std::size_t dim) {
  for (std::size_t i = 0; i < n; ++i) quiver::simd::normalize(v + i * dim, dim);
}

// ---- FlatIndex ------------------------------------------------------------------------------
void* qref_flat_new(std::size_t dim, int metric) {
  quiver::FlatIndex* out = nullptr;
  guarded([&] { out = new quiver::FlatIndex(dim, static_cast<quiver::Metric>(metric)); });
  return out;
}
void qref_flat_free(void* h) { delete static_cast<quiver::FlatIndex*>(h); }
int qref_flat_add(void* h, const float* x, std::size_t n, const std::uint64_t* labels) {
  return guarded([&] { static_cast<quiver::FlatIndex*>(h)->add(x, n, labels); });
}
int qref_flat_search(void* h, const float* q, std::size_t nq, std::size_t k,
                     const std::uint64_t* allowed, std::int64_t n_allowed, std::size_t threads,
                     std::uint64_t* out_labels, float* out_dist) {
  return guarded([&] {
    auto filter = make_filter(allowed, n_allowed);
    static_cast<quiver::FlatIndex*>(h)->search_batch(q, nq, k, out_labels, out_dist, filter.get(),
                                                     pool_for(threads));
  });
}

int qref_flat_save(void* h, const char* path) {
  return guarded([&] { static_cast<quiver::FlatIndex*>(h)->save(path); });
}
void* qref_flat_load(const char* path, int verify_checksums) {
  quiver::FlatIndex* out = nullptr;
  guarded([&] {
    quiver::LoadOptions o;
    o.verify_checksums = verify_checksums != 0;
    out = new quiver::FlatIndex(quiver::FlatIndex::load(path, o));
  });
  return out;
}
std::size_t qref_flat_size(void* h) { return static_cast<quiver::FlatIndex*>(h)->size(); }

// ---- IvfPqIndex -----------------------------------------------------------------------------
void* qref_ivfpq_new(std::size_t dim, int metric, std::size_t nlist, std::size_t m,
                     std::size_t train_iterations, int store_vectors, std::uint64_t seed) {
  quiver::IvfPqIndex* out = nullptr;
  guarded([&] {
    quiver::IvfPqParams p;
    p.dim = dim;
    p.metric = static_cast<quiver::Metric>(metric);
    p.nlist = nlist;
    p.m = m;
    p.train_iterations = train_iterations;
    p.store_vectors = store_vectors != 0;
    p.seed = seed;
    out = new quiver::IvfPqIndex(p);
  });
  return out;
}
void qref_ivfpq_free(void* h) { delete static_cast<quiver::IvfPqIndex*>(h); }
int qref_ivfpq_train(void* h, const float* x, std::size_t n, std::size_t threads) {
  return guarded([&] { static_cast<quiver::IvfPqIndex*>(h)->train(x, n, pool_for(threads)); });
}
int qref_ivfpq_add(void* h, const float* x, std::size_t n, const std::uint64_t* labels,
                   std::size_t threads) {
  return guarded(
      [&] { static_cast<quiver::IvfPqIndex*>(h)->add(x, n, labels, pool_for(threads)); });
}
int qref_ivfpq_search(void* h, const float* q, std::size_t nq, std::size_t k, std::size_t nprobe,
                      std::size_t refine_factor, const std::uint64_t* allowed,
                      std::int64_t n_allowed, std::size_t threads, std::uint64_t* out_labels,
                      float* out_dist) {
  return guarded([&] {
    auto filter = make_filter(allowed, n_allowed);
    quiver::IvfPqSearchParams p;
    p.nprobe = nprobe;
    p.refine_factor = refine_factor;
    p.filter = filter.get();
    static_cast<quiver::IvfPqIndex*>(h)->search_batch(q, nq, k, out_labels, out_dist, p,
                                                      pool_for(threads));
  });
}
int qref_ivfpq_save(void* h, const char* path) {
  return guarded([&] { static_cast<quiver::IvfPqIndex*>(h)->save(path); });
}
void* qref_ivfpq_load(const char* path, int verify_checksums) {
  quiver::IvfPqIndex* out = nullptr;
  guarded([&] {
    quiver::LoadOptions o;
    o.verify_checksums = verify_checksums != 0;
    out = new quiver::IvfPqIndex(quiver::IvfPqIndex::load(path, o));
  });
  return out;
}
std::size_t qref_ivfpq_size(void* h) { return static_cast<quiver::IvfPqIndex*>(h)->size(); }
std::size_t qref_ivfpq_memory_bytes(void* h) { return static_cast<quiver::IvfPqIndex*>(h)->memory_bytes(); }
// out[nlist]: the list sizes.
void qref_ivfpq_list_sizes(void* h, std::uint64_t* out) {
  const auto sizes = static_cast<quiver::IvfPqIndex*>(h)->list_sizes();
  for (std::size_t l = 0; l < sizes.size(); ++l) out[l] = sizes[l];
}

// ---- k-means / PQ ---------------------------------------------------------------------------
int qref_kmeans(const float* x, std::size_t n, std::size_t dim, std::size_t k,
                std::size_t iterations, std::size_t max_points_per_centroid, std::uint64_t seed,
                std::size_t threads, float* out) {
  return guarded([&] {
    quiver::KMeansParams kp;
    kp.k = k;
    kp.iterations = iterations;
    kp.max_points_per_centroid = max_points_per_centroid;
    kp.seed = seed;
    const auto c = quiver::kmeans(x, n, dim, kp, pool_for(threads));
    std::memcpy(out, c.data(), c.size() * sizeof(float));
  });
}

std::size_t qref_nearest_centroid(const float* x, const float* centroids, std::size_t k,
                                  std::size_t dim) {
  return quiver::nearest_centroid(x, centroids, k, dim);
}

// PQ with a given codebook (m x 256 x dsub): encode n vectors, or build per-query tables.
int qref_pq_encode(std::size_t dim, std::size_t m, const float* codebook, const float* x,
                   std::size_t n, std::uint8_t* codes) {
  return guarded([&] {
    quiver::ProductQuantizer pq(dim, m);
    pq.set_centroids(std::vector<float>(codebook, codebook + 256 * dim));
    for (std::size_t i = 0; i < n; ++i) pq.encode(x + i * dim, codes + i * m);
  });
}
int qref_pq_tables(std::size_t dim, std::size_t m, const float* codebook, const float* q,
                   float* l2_table, float* ip_table) {
  return guarded([&] {
    quiver::ProductQuantizer pq(dim, m);
    pq.set_centroids(std::vector<float>(codebook, codebook + 256 * dim));
    pq.compute_l2_table(q, l2_table);
    pq.compute_ip_table(q, ip_table);
  });
}
int qref_pq_adc(std::size_t dim, std::size_t m, const float* codebook, const float* table,
                const std::uint8_t* codes, std::size_t n, float* out_batch, float* out_single) {
  return guarded([&] {
    quiver::ProductQuantizer pq(dim, m);
    pq.set_centroids(std::vector<float>(codebook, codebook + 256 * dim));
    pq.adc_batch(table, codes, n, out_batch);
    for (std::size_t i = 0; i < n; ++i) out_single[i] = pq.adc(table, codes + i * m);
  });
}
int qref_pq_train(std::size_t dim, std::size_t m, const float* x, std::size_t n,
                  std::size_t iterations, std::uint64_t seed, std::size_t threads,
                  float* codebook) {
  return guarded([&] {
    quiver::ProductQuantizer pq(dim, m);
    pq.train(x, n, pool_for(threads), iterations, seed);
    std::memcpy(codebook, pq.centroids().data(), pq.centroids().size() * sizeof(float));
  });
}

}  // extern "C"
