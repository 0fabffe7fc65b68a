#include "quiver/flat_index.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <mutex>

#include "container.h"
#include "device_util.h"

namespace quiver {

namespace {

constexpr std::uint32_t kMetaSection = internal::section_tag("META");
constexpr std::uint32_t kVectorSection = internal::section_tag("VECT");
constexpr std::uint32_t kLabelSection = internal::section_tag("LABL");

/// META payload of a flat index file (src/flat_index.cc:24-29).
struct FlatFileMeta {
  std::uint64_t dim;
  std::uint64_t count;
  std::uint32_t metric;
  std::uint32_t reserved;
};
static_assert(sizeof(FlatFileMeta) == 24);

}  // namespace

using internal::check_finite;
using internal::qvh_check;

FlatIndex::FlatIndex(std::size_t dim, Metric metric) : dim_(dim), metric_(metric) {
  QUIVER_CHECK(dim >= 1 && dim <= kMaxDimension,
               "dimension must be in [1, " + std::to_string(kMaxDimension) + "]");
  QUIVER_CHECK(
      metric == Metric::kL2 || metric == Metric::kInnerProduct || metric == Metric::kCosine,
      "unknown metric");
}

void FlatIndex::add(const float* vectors, std::size_t n, const Label* labels) {
  if (n == 0) return;
  QUIVER_CHECK(vectors != nullptr, "vectors must not be null");
  check_finite(vectors, n * dim_);
  if (labels != nullptr) {
    QUIVER_CHECK(std::find(labels, labels + n, kInvalidLabel) == labels + n,
                 "label 2^64-1 is reserved (it marks empty result slots)");
  }
  std::unique_lock lock(*mu_);
  const std::size_t first = labels_.size();
  QUIVER_CHECK(first + n <= std::numeric_limits<NodeId>::max(),
               "FlatIndex holds at most 2^32 vectors");
  if (!dev_) {
    qvh_flat* h = nullptr;
    qvh_check(qvh_flat_create(static_cast<std::uint32_t>(dim_), static_cast<int>(metric_), &h),
              "FlatIndex device mirror");
    dev_ = std::shared_ptr<qvh_flat>(h, qvh_flat_destroy);
  }
  // The host copy receives the rows as stored (normalized for cosine by the device).
  const std::size_t old = data_.size();
  data_.resize(old + n * dim_);
  const qvh_status st = qvh_flat_append(dev_.get(), vectors, n, data_.data() + old);
  if (st != QVH_OK) {
    data_.resize(old);
    qvh_check(st, "FlatIndex::add");
  }
  labels_.reserve(first + n);
  for (std::size_t i = 0; i < n; ++i) labels_.push_back(labels ? labels[i] : first + i);
}

void FlatIndex::search_rows(const float* queries, std::size_t nq, std::size_t k,
                            const Filter* filter, ThreadPool* pool, Label* out_labels,
                            float* out_dist) const {
  const std::size_t n = labels_.size();
  if (n == 0) {
    std::fill(out_labels, out_labels + nq * k, kInvalidLabel);
    std::fill(out_dist, out_dist + nq * k, std::numeric_limits<float>::infinity());
    return;
  }
  QUIVER_CHECK(k <= 0xFFFFFFFFull, "k is too large");
  ThreadPool& tp = pool ? *pool : ThreadPool::global();
  std::vector<std::uint64_t> bitmap;
  if (filter != nullptr) {
    bitmap = internal::filter_bitmap(*filter, n, [&](std::size_t i) { return labels_[i]; }, tp);
  }
  std::vector<std::uint32_t> rows(nq * k);
  qvh_check(qvh_flat_search(dev_.get(), queries, nq, static_cast<std::uint32_t>(k),
                            filter ? bitmap.data() : nullptr, rows.data(), out_dist),
            "FlatIndex::search_batch");
  tp.parallel_for(nq * k, 4096, [&](std::size_t b, std::size_t e) {
    for (std::size_t i = b; i < e; ++i) {
      out_labels[i] = rows[i] == QVH_EMPTY_ROW ? kInvalidLabel : labels_[rows[i]];
    }
  });
}

std::vector<Neighbor> FlatIndex::search(const float* query, std::size_t k,
                                        const Filter* filter) const {
  QUIVER_CHECK(query != nullptr, "query must not be null");
  check_finite(query, dim_);
  std::vector<Label> labels(k);
  std::vector<float> distances(k);
  {
    std::shared_lock lock(*mu_);
    if (k > 0) search_rows(query, 1, k, filter, nullptr, labels.data(), distances.data());
  }
  std::vector<Neighbor> out;
  out.reserve(k);
  for (std::size_t j = 0; j < k && labels[j] != kInvalidLabel; ++j) {
    out.push_back({distances[j], labels[j]});
  }
  return out;
}

void FlatIndex::search_batch(const float* queries, std::size_t nq, std::size_t k, Label* labels,
                             float* distances, const Filter* filter, ThreadPool* pool) const {
  if (nq == 0 || k == 0) return;
  QUIVER_CHECK(queries != nullptr && labels != nullptr && distances != nullptr,
               "search_batch: null buffer");
  check_finite(queries, nq * dim_);
  std::shared_lock lock(*mu_);
  search_rows(queries, nq, k, filter, pool, labels, distances);
}

void FlatIndex::search_batch_device(const float* d_queries, std::size_t nq, std::size_t k,
                                    const std::uint64_t* d_row_bitmap, std::uint32_t* d_rows,
                                    float* d_distances, void* stream) const {
  if (nq == 0 || k == 0) return;
  QUIVER_CHECK(d_queries != nullptr && d_rows != nullptr && d_distances != nullptr,
               "search_batch_device: null buffer");
  QUIVER_CHECK(k <= 0xFFFFFFFFull, "k is too large");
  std::shared_lock lock(*mu_);
  QUIVER_CHECK(dev_ != nullptr && !labels_.empty(), "search_batch_device: the index is empty");
  qvh_check(qvh_flat_search_device(dev_.get(), d_queries, nq, static_cast<std::uint32_t>(k), d_row_bitmap, d_rows,
                                   d_distances, stream),
            "FlatIndex::search_batch_device");
}

void FlatIndex::search_batch_device_rows(const float* d_queries, std::size_t nq, std::size_t k,
                                         const std::uint32_t* d_row_list, std::size_t nrows, std::uint32_t* d_rows,
                                         float* d_distances, void* stream) const {
  if (nq == 0 || k == 0) return;
  QUIVER_CHECK(d_queries != nullptr && d_rows != nullptr && d_distances != nullptr,
               "search_batch_device_rows: null buffer");
  QUIVER_CHECK(k <= 0xFFFFFFFFull, "k is too large");
  std::shared_lock lock(*mu_);
  QUIVER_CHECK(dev_ != nullptr && !labels_.empty(), "search_batch_device_rows: the index is empty");
  qvh_check(qvh_flat_search_device_rows(dev_.get(), d_queries, nq, static_cast<std::uint32_t>(k), d_row_list, nrows,
                                        d_rows, d_distances, stream),
            "FlatIndex::search_batch_device_rows");
}

std::vector<std::uint64_t> FlatIndex::row_bitmap(const Filter& filter) const {
  std::shared_lock lock(*mu_);
  return internal::filter_bitmap(filter, labels_.size(), [&](std::size_t i) { return labels_[i]; },
                                 ThreadPool::global());
}

std::vector<Label> FlatIndex::labels() const {
  std::shared_lock lock(*mu_);
  return labels_;
}

std::size_t FlatIndex::size() const {
  std::shared_lock lock(*mu_);
  return labels_.size();
}

void FlatIndex::save(const std::string& path) const {
  std::shared_lock lock(*mu_);
  internal::ContainerWriter w(internal::ContainerKind::kFlat);
  w.section_pod(kMetaSection, FlatFileMeta{dim_, labels_.size(), static_cast<std::uint32_t>(metric_), 0});
  w.section_bytes(kVectorSection, data_.data(), data_.size() * sizeof(float));
  w.section_bytes(kLabelSection, labels_.data(), labels_.size() * sizeof(Label));
  w.commit(path);
}

FlatIndex FlatIndex::load(const std::string& path, const LoadOptions& options) {
  const auto img = internal::ContainerImage::open(path, internal::ContainerKind::kFlat, options.verify_checksums);
  const std::string bad = "corrupt index file '" + path + "': ";
  const auto meta = img->pod<FlatFileMeta>(kMetaSection);
  QUIVER_CHECK(meta.dim >= 1 && meta.dim <= kMaxDimension, bad + "bad dimension");
  QUIVER_CHECK(meta.metric <= static_cast<std::uint32_t>(Metric::kCosine), bad + "unknown metric");
  QUIVER_CHECK(meta.count <= img->file_size() / (meta.dim * sizeof(float) + sizeof(Label)), bad + "bad vector count");
  const std::size_t dim = static_cast<std::size_t>(meta.dim), count = static_cast<std::size_t>(meta.count);
  QUIVER_CHECK(count <= std::numeric_limits<NodeId>::max(), "FlatIndex holds at most 2^32 vectors");
  const float* vectors = img->array<float>(kVectorSection, count * dim);
  const Label* labels = img->array<Label>(kLabelSection, count);
  QUIVER_CHECK(std::all_of(vectors, vectors + count * dim, [](float v) { return std::isfinite(v); }),
               bad + "non-finite vector values");
  FlatIndex index(dim, static_cast<Metric>(meta.metric));
  if (count > 0) {
    qvh_flat* h = nullptr;
    qvh_check(qvh_flat_create(static_cast<std::uint32_t>(dim), static_cast<int>(meta.metric), &h),
              "FlatIndex device mirror");
    index.dev_ = std::shared_ptr<qvh_flat>(h, qvh_flat_destroy);
    // The file holds rows as stored (already normalized for cosine): upload them unchanged.
    qvh_check(qvh_flat_append_stored(h, vectors, count), "FlatIndex::load");
  }
  index.data_.assign(vectors, vectors + count * dim);
  index.labels_.assign(labels, labels + count);
  return index;
}

}  // namespace quiver
