#include "quiver/ivfpq_index.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <mutex>
#include <random>
#include <shared_mutex>

#include "container.h"
#include "device_util.h"
#include "quiver/quantizer.h"

namespace quiver {

namespace {

using internal::check_finite;
using internal::qvh_check;

constexpr std::size_t kMaxLists = std::size_t{1} << 24;
constexpr std::size_t kSubCentroids = 256;
/// The precomputed L2 term table is used when it fits this budget (src/ivfpq_index.cc:73-74).
constexpr std::size_t kMaxPrecomputedBytes = std::size_t{256} << 20;

constexpr std::uint32_t kMetaSection = internal::section_tag("META");
constexpr std::uint32_t kCentroidSection = internal::section_tag("CENT");
constexpr std::uint32_t kCodebookSection = internal::section_tag("PQCB");
constexpr std::uint32_t kOffsetSection = internal::section_tag("LOFF");
constexpr std::uint32_t kCodeSection = internal::section_tag("CODE");
constexpr std::uint32_t kLabelSection = internal::section_tag("LABL");
constexpr std::uint32_t kVectorSection = internal::section_tag("VECT");

/// META payload of an IVF-PQ index file (src/ivfpq_index.cc:32-43).
struct IvfPqFileMeta {
  std::uint64_t dim, nlist, m, count, train_iterations, seed;
  std::uint32_t metric, store_vectors, trained, reserved;
};
static_assert(sizeof(IvfPqFileMeta) == 64);

void normalize_rows(float* v, std::size_t n, std::size_t dim) {
  if (n == 0) return;
  qvh_check(qvh_normalize(v, n, static_cast<std::uint32_t>(dim)), "normalize");
}

struct PointsDeleter {
  void operator()(qvh_points* p) const noexcept { qvh_points_destroy(p); }
};

/// Nearest centroid of every row, CentroidTable::nearest_batch arithmetic, on the device.
std::vector<std::uint32_t> nearest(const float* x, std::size_t n, std::size_t dim, const float* cent,
                                   std::size_t k, bool max_ip) {
  qvh_points* raw = nullptr;
  qvh_check(qvh_points_create(x, n, static_cast<std::uint32_t>(dim), &raw), "assign");
  std::unique_ptr<qvh_points, PointsDeleter> pts(raw);
  std::vector<std::uint32_t> out(n);
  qvh_check(qvh_points_nearest(pts.get(), cent, static_cast<std::uint32_t>(k), max_ip ? 1 : 0, out.data()),
            "assign");
  return out;
}

}  // namespace

struct IvfPqIndex::Impl {
  IvfPqParams params;
  std::shared_ptr<qvh_ivfpq> dev;
  std::vector<float> centroids;  // nlist x dim
  std::vector<float> codebook;   // m x 256 x dsub
  bool use_precomputed = false;
  std::vector<std::uint64_t> offsets;  // nlist + 1, CSR over lists
  std::vector<Label> labels;           // CSR order
  std::size_t count = 0;
  mutable std::shared_mutex mu;
  bool trained = false;

  explicit Impl(const IvfPqParams& p) : params(p) {
    QUIVER_CHECK(p.dim >= 1 && p.dim <= kMaxDimension,
                 "dimension must be in [1, " + std::to_string(kMaxDimension) + "]");
    QUIVER_CHECK(p.nlist >= 1 && p.nlist <= kMaxLists, "nlist must be in [1, 2^24]");
    QUIVER_CHECK(p.m > 0 && p.dim % p.m == 0, "PQ: dimension " + std::to_string(p.dim) +
                                                  " must be divisible by m=" + std::to_string(p.m));
    QUIVER_CHECK(
        p.metric == Metric::kL2 || p.metric == Metric::kInnerProduct || p.metric == Metric::kCosine,
        "unknown metric");
    offsets.assign(p.nlist + 1, 0);
  }

  bool assign_by_ip() const noexcept { return params.metric == Metric::kInnerProduct; }
  bool precompute_applies() const noexcept {
    return params.metric == Metric::kL2 &&
           params.nlist * params.m * kSubCentroids * sizeof(float) <= kMaxPrecomputedBytes;
  }

  /// Creates the device handle and installs the trained state; caller holds `mu` exclusively.
  void commit(std::vector<float> cent, std::vector<float> cb) {
    qvh_ivfpq* h = nullptr;
    qvh_check(qvh_ivfpq_create(static_cast<std::uint32_t>(params.dim), static_cast<int>(params.metric),
                               static_cast<std::uint32_t>(params.nlist), static_cast<std::uint32_t>(params.m),
                               params.store_vectors ? 1 : 0, &h),
              "IVF-PQ device state");
    std::shared_ptr<qvh_ivfpq> handle(h, qvh_ivfpq_destroy);
    const bool pre = precompute_applies();
    qvh_check(qvh_ivfpq_set_trained(h, cent.data(), cb.data(), pre ? 1 : 0), "IVF-PQ device state");
    dev = std::move(handle);
    centroids = std::move(cent);
    codebook = std::move(cb);
    use_precomputed = pre;
    trained = true;
  }

  // Impl::train of the reference (src/ivfpq_index.cc:144-206), with every assignment step on
  // the device: coarse k-means, residuals to the nearest cell, a random 65,536-row subset
  // (mt19937_64 seeded with seed + 2), one 256-way k-means per sub-space (seeds seed + 1 + j).
  void train(const float* in, std::size_t n, ThreadPool* pool) {
    QUIVER_CHECK(n >= params.nlist && n >= kSubCentroids,
                 "IVF-PQ training needs at least max(nlist, 256) vectors");
    check_finite(in, n * params.dim);
    {
      std::shared_lock lock(mu);
      QUIVER_CHECK(!trained, "index is already trained");
    }
    const std::size_t d = params.dim, m = params.m, dsub = d / m;
    std::vector<float> data(in, in + n * d);
    if (params.metric == Metric::kCosine) normalize_rows(data.data(), n, d);
    KMeansParams kp;
    kp.k = params.nlist;
    kp.iterations = params.train_iterations;
    kp.seed = params.seed;
    std::vector<float> cent = kmeans(data.data(), n, d, kp, pool);
    if (params.metric == Metric::kCosine) normalize_rows(cent.data(), params.nlist, d);

    const std::vector<std::uint32_t> cell = nearest(data.data(), n, d, cent.data(), params.nlist, assign_by_ip());
    std::vector<float> residuals(n * d);
    for (std::size_t i = 0; i < n; ++i) {
      const float* x = data.data() + i * d;
      const float* c = cent.data() + static_cast<std::size_t>(cell[i]) * d;
      for (std::size_t j = 0; j < d; ++j) residuals[i * d + j] = x[j] - c[j];
    }
    const std::size_t pq_n = std::min<std::size_t>(n, 65536);
    if (pq_n < n) {
      std::mt19937_64 rng(params.seed + 2);
      for (std::size_t i = 0; i < pq_n; ++i) {
        const std::size_t j = i + rng() % (n - i);
        std::swap_ranges(residuals.begin() + static_cast<std::ptrdiff_t>(i * d),
                         residuals.begin() + static_cast<std::ptrdiff_t>((i + 1) * d),
                         residuals.begin() + static_cast<std::ptrdiff_t>(j * d));
      }
    }
    std::vector<float> cb(m * kSubCentroids * dsub);
    std::vector<float> sub(pq_n * dsub);
    for (std::size_t j = 0; j < m; ++j) {
      for (std::size_t i = 0; i < pq_n; ++i) {
        std::memcpy(sub.data() + i * dsub, residuals.data() + i * d + j * dsub, dsub * sizeof(float));
      }
      KMeansParams sp;
      sp.k = kSubCentroids;
      sp.iterations = params.train_iterations;
      sp.seed = params.seed + 1 + j;
      const std::vector<float> c = kmeans(sub.data(), pq_n, dsub, sp, pool);
      std::copy(c.begin(), c.end(), cb.begin() + static_cast<std::ptrdiff_t>(j * kSubCentroids * dsub));
    }
    std::unique_lock lock(mu);
    QUIVER_CHECK(!trained, "index is already trained");
    commit(std::move(cent), std::move(cb));
  }

  // Impl::add of the reference (src/ivfpq_index.cc:208-271). The encode runs on the device without
  // the index lock (the trained state it reads never changes once set; the reference likewise
  // only observes `trained` under the shared lock), so searches proceed meanwhile; the exclusive
  // lock is taken only to append the encoded entries and place their labels.
  void add(const float* in, std::size_t n, const Label* new_labels) {
    if (n == 0) return;
    check_finite(in, n * params.dim);
    if (new_labels != nullptr) {
      QUIVER_CHECK(std::find(new_labels, new_labels + n, kInvalidLabel) == new_labels + n,
                   "label 2^64-1 is reserved (it marks empty result slots)");
    }
    {
      std::shared_lock lock(mu);
      QUIVER_CHECK(trained, "IVF-PQ index must be trained before add()");
    }
    std::vector<std::uint32_t> assign(n);
    std::vector<std::uint8_t> codes(n * params.m);
    std::vector<float> stored(params.store_vectors ? n * params.dim : 0);
    qvh_check(qvh_ivfpq_encode(dev.get(), in, n, assign.data(), codes.data(),
                               params.store_vectors ? stored.data() : nullptr),
              "IvfPqIndex::add");

    std::unique_lock lock(mu);
    qvh_check(qvh_ivfpq_append(dev.get(), assign.data(), codes.data(),
                               params.store_vectors ? stored.data() : nullptr, n),
              "IvfPqIndex::add");
    // The device appended each vector after its list's entries in input order; place the
    // labels the same way (src/ivfpq_index.cc:263-269).
    const std::size_t nl = params.nlist;
    std::vector<std::uint64_t> added(nl, 0);
    for (std::uint32_t l : assign) ++added[l];
    std::vector<std::uint64_t> next(nl + 1, 0);
    for (std::size_t l = 0; l < nl; ++l) next[l + 1] = next[l] + (offsets[l + 1] - offsets[l]) + added[l];
    std::vector<Label> merged(count + n);
    std::vector<std::uint64_t> cursor(nl);
    for (std::size_t l = 0; l < nl; ++l) {
      const std::uint64_t len = offsets[l + 1] - offsets[l];
      std::copy(labels.begin() + static_cast<std::ptrdiff_t>(offsets[l]),
                labels.begin() + static_cast<std::ptrdiff_t>(offsets[l] + len),
                merged.begin() + static_cast<std::ptrdiff_t>(next[l]));
      cursor[l] = next[l] + len;
    }
    for (std::size_t i = 0; i < n; ++i) merged[cursor[assign[i]]++] = new_labels ? new_labels[i] : count + i;
    labels = std::move(merged);
    offsets = std::move(next);
    count += n;
  }

  void search_rows(const float* queries, std::size_t nq, std::size_t k, const IvfPqSearchParams& p,
                   ThreadPool* pool, Label* out_labels, float* out_dist) const {
    std::fill(out_labels, out_labels + nq * k, kInvalidLabel);
    std::fill(out_dist, out_dist + nq * k, std::numeric_limits<float>::infinity());
    if (!trained || count == 0) return;
    ThreadPool& tp = pool ? *pool : ThreadPool::global();
    std::vector<std::uint64_t> bitmap;
    if (p.filter != nullptr) {
      bitmap = internal::filter_bitmap(*p.filter, count, [&](std::size_t i) { return labels[i]; }, tp);
    }
    QUIVER_CHECK(k <= 0xFFFFFFFFull, "k is too large");
    const std::uint32_t nprobe =
        static_cast<std::uint32_t>(std::min<std::size_t>(std::max<std::size_t>(p.nprobe, 1), params.nlist));
    std::vector<std::uint64_t> refs(nq * k);
    qvh_check(qvh_ivfpq_search(dev.get(), queries, nq, static_cast<std::uint32_t>(k), nprobe, p.refine_factor,
                               p.filter ? bitmap.data() : nullptr, refs.data(), out_dist),
              "IvfPqIndex::search_batch");
    tp.parallel_for(nq * k, 4096, [&](std::size_t b, std::size_t e) {
      for (std::size_t i = b; i < e; ++i) {
        const std::uint64_t ref = refs[i];
        out_labels[i] = ref == QVH_EMPTY_REF ? kInvalidLabel : labels[offsets[ref >> 32] + (ref & 0xFFFFFFFFull)];
      }
    });
  }
};

IvfPqIndex::IvfPqIndex(const IvfPqParams& params) : impl_(std::make_unique<Impl>(params)) {}
IvfPqIndex::IvfPqIndex(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
IvfPqIndex::~IvfPqIndex() = default;
IvfPqIndex::IvfPqIndex(IvfPqIndex&&) noexcept = default;
IvfPqIndex& IvfPqIndex::operator=(IvfPqIndex&&) noexcept = default;

void IvfPqIndex::train(const float* vectors, std::size_t n, ThreadPool* pool) {
  QUIVER_CHECK(vectors != nullptr, "vectors must not be null");
  impl_->train(vectors, n, pool);
}

bool IvfPqIndex::is_trained() const noexcept {
  std::shared_lock lock(impl_->mu);
  return impl_->trained;
}

void IvfPqIndex::add(const float* vectors, std::size_t n, const Label* labels, ThreadPool* /*pool*/) {
  QUIVER_CHECK(vectors != nullptr || n == 0, "vectors must not be null");
  impl_->add(vectors, n, labels);
}

std::vector<Neighbor> IvfPqIndex::search(const float* query, std::size_t k,
                                         const IvfPqSearchParams& params) const {
  QUIVER_CHECK(query != nullptr, "query must not be null");
  check_finite(query, impl_->params.dim);
  std::vector<Label> labels(k);
  std::vector<float> dist(k);
  if (k > 0) {
    std::shared_lock lock(impl_->mu);
    impl_->search_rows(query, 1, k, params, nullptr, labels.data(), dist.data());
  }
  std::vector<Neighbor> out;
  for (std::size_t j = 0; j < k && labels[j] != kInvalidLabel; ++j) out.push_back({dist[j], labels[j]});
  return out;
}

void IvfPqIndex::search_batch(const float* queries, std::size_t nq, std::size_t k, Label* labels,
                              float* distances, const IvfPqSearchParams& params, ThreadPool* pool) const {
  if (nq == 0 || k == 0) return;
  QUIVER_CHECK(queries != nullptr && labels != nullptr && distances != nullptr, "search_batch: null buffer");
  check_finite(queries, nq * impl_->params.dim);
  std::shared_lock lock(impl_->mu);
  impl_->search_rows(queries, nq, k, params, pool, labels, distances);
}

void IvfPqIndex::search_batch_device(const float* d_queries, std::size_t nq, std::size_t k,
                                     const IvfPqSearchParams& params, const std::uint64_t* d_position_bitmap,
                                     std::uint64_t* d_refs, float* d_distances, void* stream) const {
  if (nq == 0 || k == 0) return;
  QUIVER_CHECK(d_queries != nullptr && d_refs != nullptr && d_distances != nullptr,
               "search_batch_device: null buffer");
  QUIVER_CHECK(k <= 0xFFFFFFFFull, "k is too large");
  std::shared_lock lock(impl_->mu);
  QUIVER_CHECK(impl_->trained && impl_->count > 0, "search_batch_device: the index is untrained or empty");
  const std::uint32_t nprobe = static_cast<std::uint32_t>(
      std::min<std::size_t>(std::max<std::size_t>(params.nprobe, 1), impl_->params.nlist));
  qvh_check(qvh_ivfpq_search_device(impl_->dev.get(), d_queries, nq, static_cast<std::uint32_t>(k), nprobe,
                                    params.refine_factor, d_position_bitmap, d_refs, d_distances,
                                    stream),
            "IvfPqIndex::search_batch_device");
}

std::vector<std::uint64_t> IvfPqIndex::position_bitmap(const Filter& filter) const {
  std::shared_lock lock(impl_->mu);
  return internal::filter_bitmap(filter, impl_->count, [&](std::size_t i) { return impl_->labels[i]; },
                                 ThreadPool::global());
}

std::size_t IvfPqIndex::size() const noexcept {
  std::shared_lock lock(impl_->mu);
  return impl_->count;
}
std::size_t IvfPqIndex::dim() const noexcept { return impl_->params.dim; }
const IvfPqParams& IvfPqIndex::params() const noexcept { return impl_->params; }

std::size_t IvfPqIndex::memory_bytes() const noexcept {
  std::shared_lock lock(impl_->mu);
  const Impl& ix = *impl_;
  const std::size_t pre = ix.use_precomputed ? ix.params.nlist * ix.params.m * kSubCentroids : 0;
  std::size_t bytes = (ix.centroids.size() + ix.codebook.size() + pre) * sizeof(float);
  bytes += ix.count * ix.params.m + ix.count * sizeof(Label);
  if (ix.params.store_vectors) bytes += ix.count * ix.params.dim * sizeof(float);
  return bytes;
}

std::vector<std::size_t> IvfPqIndex::list_sizes() const {
  std::shared_lock lock(impl_->mu);
  std::vector<std::size_t> out(impl_->params.nlist);
  for (std::size_t l = 0; l < out.size(); ++l) out[l] = impl_->offsets[l + 1] - impl_->offsets[l];
  return out;
}

std::vector<float> IvfPqIndex::centroids() const {
  std::shared_lock lock(impl_->mu);
  return impl_->centroids;
}

std::vector<float> IvfPqIndex::codebook() const {
  std::shared_lock lock(impl_->mu);
  return impl_->codebook;
}

void IvfPqIndex::set_trained(const float* centroids, const float* codebook) {
  QUIVER_CHECK(centroids != nullptr && codebook != nullptr, "set_trained: null state");
  const auto& p = impl_->params;
  const std::size_t nc = p.nlist * p.dim, nb = p.m * kSubCentroids * (p.dim / p.m);
  check_finite(centroids, nc);
  check_finite(codebook, nb);
  std::unique_lock lock(impl_->mu);
  QUIVER_CHECK(!impl_->trained, "index is already trained");
  impl_->commit(std::vector<float>(centroids, centroids + nc), std::vector<float>(codebook, codebook + nb));
}

std::vector<std::uint64_t> IvfPqIndex::list_offsets() const {
  std::shared_lock lock(impl_->mu);
  return impl_->offsets;
}

std::vector<Label> IvfPqIndex::list_labels() const {
  std::shared_lock lock(impl_->mu);
  return impl_->labels;
}

std::vector<std::uint8_t> IvfPqIndex::list_codes() const {
  std::shared_lock lock(impl_->mu);
  std::vector<std::uint8_t> out(impl_->count * impl_->params.m);
  if (impl_->count) qvh_check(qvh_ivfpq_lists(impl_->dev.get(), out.data(), nullptr), "list_codes");
  return out;
}

std::vector<float> IvfPqIndex::list_vectors() const {
  std::shared_lock lock(impl_->mu);
  QUIVER_CHECK(impl_->params.store_vectors, "vectors are not stored (store_vectors is off)");
  std::vector<float> out(impl_->count * impl_->params.dim);
  if (impl_->count) qvh_check(qvh_ivfpq_lists(impl_->dev.get(), nullptr, out.data()), "list_vectors");
  return out;
}

qvh_ivfpq* IvfPqIndex::device_handle() const noexcept { return impl_->dev.get(); }

void IvfPqIndex::save(const std::string& path) const {
  std::shared_lock lock(impl_->mu);
  const Impl& ix = *impl_;
  const IvfPqParams& p = ix.params;
  const IvfPqFileMeta meta{p.dim, p.nlist, p.m, ix.count, p.train_iterations, p.seed,
                           static_cast<std::uint32_t>(p.metric), p.store_vectors ? 1u : 0u,
                           ix.trained ? 1u : 0u, 0};
  // Codes and vectors live on the device; bring them back in list (CSR) order.
  std::vector<std::uint8_t> codes(ix.count * p.m);
  std::vector<float> vectors(p.store_vectors ? ix.count * p.dim : 0);
  if (ix.count > 0) {
    qvh_check(qvh_ivfpq_lists(ix.dev.get(), codes.data(), p.store_vectors ? vectors.data() : nullptr),
              "IvfPqIndex::save");
  }
  internal::ContainerWriter w(internal::ContainerKind::kIvfPq);
  w.section_pod(kMetaSection, meta);
  w.section_bytes(kCentroidSection, ix.centroids.data(), ix.centroids.size() * sizeof(float));
  w.section_bytes(kCodebookSection, ix.codebook.data(), ix.codebook.size() * sizeof(float));
  w.section_bytes(kOffsetSection, ix.offsets.data(), ix.offsets.size() * sizeof(std::uint64_t));
  w.section_bytes(kCodeSection, codes.data(), codes.size());
  w.section_bytes(kLabelSection, ix.labels.data(), ix.labels.size() * sizeof(Label));
  if (p.store_vectors) w.section_bytes(kVectorSection, vectors.data(), vectors.size() * sizeof(float));
  w.commit(path);
}

IvfPqIndex IvfPqIndex::load(const std::string& path, const LoadOptions& options) {
  const auto img = internal::ContainerImage::open(path, internal::ContainerKind::kIvfPq, options.verify_checksums);
  const std::string bad = "corrupt index file '" + path + "': ";
  const auto meta = img->pod<IvfPqFileMeta>(kMetaSection);
  QUIVER_CHECK(meta.dim >= 1 && meta.dim <= kMaxDimension, bad + "bad dimension");
  QUIVER_CHECK(meta.m >= 1 && meta.m <= meta.dim && meta.dim % meta.m == 0, bad + "bad m");
  QUIVER_CHECK(meta.nlist >= 1 && meta.nlist <= kMaxLists, bad + "bad nlist");
  QUIVER_CHECK((meta.nlist + 1) * sizeof(std::uint64_t) <= img->file_size(), bad + "bad nlist");
  QUIVER_CHECK(meta.metric <= static_cast<std::uint32_t>(Metric::kCosine), bad + "bad metric");
  QUIVER_CHECK(meta.count <= img->file_size(), bad + "bad count");
  IvfPqParams p;
  p.dim = static_cast<std::size_t>(meta.dim);
  p.nlist = static_cast<std::size_t>(meta.nlist);
  p.m = static_cast<std::size_t>(meta.m);
  p.train_iterations = static_cast<std::size_t>(meta.train_iterations);
  p.seed = meta.seed;
  p.metric = static_cast<Metric>(meta.metric);
  p.store_vectors = meta.store_vectors != 0;
  auto impl = std::make_unique<Impl>(p);
  const std::size_t count = static_cast<std::size_t>(meta.count);
  const std::uint64_t* offsets = img->array<std::uint64_t>(kOffsetSection, p.nlist + 1);
  QUIVER_CHECK(offsets[0] == 0 && offsets[p.nlist] == count, bad + "bad list offsets");
  for (std::size_t l = 0; l < p.nlist; ++l) QUIVER_CHECK(offsets[l] <= offsets[l + 1], bad + "bad list offsets");
  const std::uint8_t* codes = img->array<std::uint8_t>(kCodeSection, count * p.m);
  const Label* labels = img->array<Label>(kLabelSection, count);
  const float* vectors = nullptr;
  if (p.store_vectors) {
    vectors = img->array<float>(kVectorSection, count * p.dim);
    QUIVER_CHECK(std::all_of(vectors, vectors + count * p.dim, [](float v) { return std::isfinite(v); }),
                 bad + "non-finite stored vectors");
  }
  if (meta.trained != 0) {
    const std::size_t nc = p.nlist * p.dim, nb = p.m * kSubCentroids * (p.dim / p.m);
    const float* cent = img->array<float>(kCentroidSection, nc);
    const float* cb = img->array<float>(kCodebookSection, nb);
    const auto finite = [](float v) { return std::isfinite(v); };
    QUIVER_CHECK(std::all_of(cent, cent + nc, finite) && std::all_of(cb, cb + nb, finite),
                 bad + "non-finite centroids");
    impl->commit(std::vector<float>(cent, cent + nc), std::vector<float>(cb, cb + nb));
    if (count > 0) qvh_check(qvh_ivfpq_set_lists(impl->dev.get(), offsets, codes, vectors), "IvfPqIndex::load");
  } else {
    QUIVER_CHECK(count == 0, bad + "untrained index with vectors");
  }
  impl->offsets.assign(offsets, offsets + p.nlist + 1);
  impl->labels.assign(labels, labels + count);
  impl->count = count;
  return IvfPqIndex(std::move(impl));
}

}  // namespace quiver
