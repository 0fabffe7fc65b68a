// IVF-PQ with the reference's public API (include/quiver/ivfpq_index.h:26-81): a coarse k-means
// splits space into `nlist` cells; each vector is stored in its cell as the PQ code of its
// residual. Encoding on add and the whole query path (coarse scores, probe selection, ADC tables,
// list scan, top-k, exact re-ranking) run on the GPU through the qvh C-ABI; the lists live in
// device memory in CSR order and the labels stay on the host.
//
// Concurrency: all methods are thread-safe; searches run concurrently, add() is exclusive.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "quiver/common.h"
#include "quiver/filter.h"
#include "quiver/thread_pool.h"

struct qvh_ivfpq;

namespace quiver {

struct IvfPqParams {
  std::size_t dim = 0;
  Metric metric = Metric::kL2;
  std::size_t nlist = 1024;
  std::size_t m = 16;  ///< PQ sub-quantizers (bytes per vector); must divide dim
  std::size_t train_iterations = 20;
  /// Keep float32 copies of the vectors so results can be re-ranked exactly.
  bool store_vectors = false;
  std::uint64_t seed = 1234;
};

struct IvfPqSearchParams {
  std::size_t nprobe = 16;
  /// With store_vectors, re-rank the best k * refine_factor ADC candidates exactly (0 = off).
  std::size_t refine_factor = 0;
  const Filter* filter = nullptr;
};

class IvfPqIndex {
 public:
  explicit IvfPqIndex(const IvfPqParams& params);
  ~IvfPqIndex();
  IvfPqIndex(IvfPqIndex&&) noexcept;
  IvfPqIndex& operator=(IvfPqIndex&&) noexcept;

  /// Learns coarse centroids and residual PQ codebooks; needs n >= max(nlist, 256); once only.
  void train(const float* vectors, std::size_t n, ThreadPool* pool = nullptr);
  bool is_trained() const noexcept;

  /// `labels` may be null (labels become size() + i).
  void add(const float* vectors, std::size_t n, const Label* labels = nullptr,
           ThreadPool* pool = nullptr);

  std::vector<Neighbor> search(const float* query, std::size_t k,
                               const IvfPqSearchParams& params = {}) const;
  void search_batch(const float* queries, std::size_t nq, std::size_t k, Label* labels,
                    float* distances, const IvfPqSearchParams& params = {},
                    ThreadPool* pool = nullptr) const;

  /// Writes the index as a `.qvr` file readable by the reference's IvfPqIndex::load
  /// (src/ivfpq_index.cc:465-505); atomic replace of `path`.
  void save(const std::string& path) const;
  /// Reads a `.qvr` IVF-PQ index (src/ivfpq_index.cc:507-576): the trained state goes to the
  /// device as after train(), the CSR lists straight into the device list layout.
  static IvfPqIndex load(const std::string& path, const LoadOptions& options = {});

  std::size_t size() const noexcept;
  std::size_t dim() const noexcept;
  const IvfPqParams& params() const noexcept;
  /// Bytes of centroids, codebook, precomputed table, codes, labels and stored vectors (the
  /// reference's accounting, src/ivfpq_index.cc:446-455).
  std::size_t memory_bytes() const noexcept;
  std::vector<std::size_t> list_sizes() const;

  /// Trained state: coarse centroids [nlist][dim] and PQ codebook [m][256][dim/m].
  std::vector<float> centroids() const;
  std::vector<float> codebook() const;
  /// Installs a trained state instead of training (as loading a saved index does).
  void set_trained(const float* centroids, const float* codebook);
  /// Lists in CSR order: offsets [nlist + 1], labels, codes [size][m], vectors [size][dim].
  std::vector<std::uint64_t> list_offsets() const;
  std::vector<Label> list_labels() const;
  std::vector<std::uint8_t> list_codes() const;
  std::vector<float> list_vectors() const;
  /// The device handle (null before training), for device-resident query batches.
  qvh_ivfpq* device_handle() const noexcept;

  /// Device-resident batch (no reference counterpart; for callers whose queries already live in
  /// HBM): queries [nq][dim], the position bitmap of position_bitmap() or null (params.filter is
  /// not read), and outputs refs [nq][k] ((list << 32) | offset, all ones = empty) and distances
  /// [nq][k] are device pointers; enqueued on `stream` (a hipStream_t, null = the index's own)
  /// under the shared lock and not waited for. Queries must be finite (the caller checks); refs
  /// map to labels through list_offsets() and list_labels().
  void search_batch_device(const float* d_queries, std::size_t nq, std::size_t k,
                           const IvfPqSearchParams& params, const std::uint64_t* d_position_bitmap,
                           std::uint64_t* d_refs, float* d_distances, void* stream = nullptr) const;
  /// The filter as bits over CSR positions (bit p = list_labels()[p] admitted).
  std::vector<std::uint64_t> position_bitmap(const Filter& filter) const;

 private:
  struct Impl;
  explicit IvfPqIndex(std::unique_ptr<Impl> impl);
  std::unique_ptr<Impl> impl_;
};

}  // namespace quiver
