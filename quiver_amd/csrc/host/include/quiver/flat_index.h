// Exact brute-force index with the reference's public API (include/quiver/flat_index.h:19-58).
// Rows live twice: in host memory (vector(i), save) and in a device-resident mirror that the
// gfx950 scan reads (qvh_flat_* in include/qvh.h). search_batch is one device call per batch.
//
// Thread-safe: searches run concurrently; add() takes an exclusive lock.
#pragma once

#include <cstddef>
#include <memory>
#include <shared_mutex>
#include <string>
#include <vector>

#include "quiver/common.h"
#include "quiver/filter.h"
#include "quiver/thread_pool.h"

struct qvh_flat;

namespace quiver {

class FlatIndex {
 public:
  explicit FlatIndex(std::size_t dim, Metric metric = Metric::kL2);

  /// Appends `n` row-major vectors. `labels` may be null, in which case vector i gets label
  /// size() + i. Labels are not checked for uniqueness. Holds at most 2^32 - 1 vectors.
  void add(const float* vectors, std::size_t n, const Label* labels = nullptr);

  /// Exact k nearest neighbors, closest first; fewer than k if the index (or filter) has fewer.
  std::vector<Neighbor> search(const float* query, std::size_t k,
                               const Filter* filter = nullptr) const;

  /// Searches `nq` row-major queries on the device. Writes nq * k results; unfilled slots get
  /// kInvalidLabel and +infinity. `pool` runs the host-side filter materialization.
  void search_batch(const float* queries, std::size_t nq, std::size_t k, Label* labels,
                    float* distances, const Filter* filter = nullptr,
                    ThreadPool* pool = nullptr) const;

  std::size_t size() const;
  std::size_t dim() const noexcept { return dim_; }
  Metric metric() const noexcept { return metric_; }

  /// Writes the index as a `.qvr` file readable by the reference's FlatIndex::load
  /// (src/flat_index.cc:147-153); atomic replace of `path`.
  void save(const std::string& path) const;
  /// Reads a `.qvr` flat index (src/flat_index.cc:155-176) and uploads its rows as stored.
  static FlatIndex load(const std::string& path, const LoadOptions& options = {});

  /// Stored vector `i` (normalized for cosine). Not synchronized with add().
  const float* vector(std::size_t i) const noexcept { return data_.data() + i * dim_; }
  Label label(std::size_t i) const noexcept { return labels_[i]; }

  /// The device mirror (null before the first add); for callers that search device-resident
  /// query batches through qvh_flat_search_device.
  qvh_flat* device_handle() const noexcept { return dev_.get(); }

  /// Device-resident batch (no reference counterpart; for callers whose queries already live in
  /// HBM): queries [nq][dim], the row bitmap of row_bitmap() or null, and outputs rows [nq][k]
  /// (0xFFFFFFFF = empty) and distances [nq][k] are device pointers; the search is enqueued on
  /// `stream` (a hipStream_t, null = the index's own) under the shared lock and not waited for.
  /// Queries must be finite (the caller checks); rows map to labels through labels().
  void search_batch_device(const float* d_queries, std::size_t nq, std::size_t k,
                           const std::uint64_t* d_row_bitmap, std::uint32_t* d_rows,
                           float* d_distances, void* stream = nullptr) const;
  /// search_batch_device with the admitted rows as a device list (ascending, no repeats, each
  /// below size()) instead of a bitmap: the scan reads only the listed rows.
  void search_batch_device_rows(const float* d_queries, std::size_t nq, std::size_t k,
                                const std::uint32_t* d_row_list, std::size_t nrows, std::uint32_t* d_rows,
                                float* d_distances, void* stream = nullptr) const;
  /// The filter as bits over rows (bit i = labels()[i] admitted), as search_batch builds it.
  std::vector<std::uint64_t> row_bitmap(const Filter& filter) const;
  /// Labels by row.
  std::vector<Label> labels() const;

 private:
  void search_rows(const float* queries, std::size_t nq, std::size_t k, const Filter* filter,
                   ThreadPool* pool, Label* labels, float* distances) const;

  std::size_t dim_;
  Metric metric_;
  std::vector<float> data_;
  std::vector<Label> labels_;
  std::shared_ptr<qvh_flat> dev_;
  std::unique_ptr<std::shared_mutex> mu_ = std::make_unique<std::shared_mutex>();  // movable
};

}  // namespace quiver
