// pybind11 bindings with the reference's binding surface (python/quiver_ext.cc:24-389, nanobind
// there; nanobind is not available in this toolchain). Argument normalization happens in Python
// (quiver_amd/__init__.py); every compute call releases the GIL.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <algorithm>
#include <cstring>
#include <utility>
#include <vector>
#include <memory>
#include <mutex>

#include "qvh.h"
#include "quiver/filter.h"
#include "quiver/flat_index.h"
#include "quiver/ivfpq_index.h"
#include "quiver/quantizer.h"

namespace py = pybind11;

namespace {

using FloatMatrix = py::array_t<float, py::array::c_style>;
using LabelArray = py::array_t<std::uint64_t, py::array::c_style>;

/// Host thread pools the Python calls may ask for. num_threads = 0 is the process-wide pool; any
/// other size is created on first request and kept for the life of the module, so repeated calls
/// with one size reuse its threads (python/quiver_ext.cc:28-37 keeps one per size too).
class PoolRegistry {
 public:
  static constexpr std::size_t kMaxThreads = 1024;

  static quiver::ThreadPool* get(std::size_t threads) {
    if (threads == 0) return &quiver::ThreadPool::global();
    if (threads > kMaxThreads) throw py::value_error("num_threads must be at most 1024");
    static PoolRegistry registry;
    std::lock_guard<std::mutex> lock(registry.mu_);
    for (const auto& entry : registry.pools_) {
      if (entry.first == threads) return entry.second.get();
    }
    registry.pools_.emplace_back(threads, std::make_unique<quiver::ThreadPool>(threads));
    return registry.pools_.back().second.get();
  }

 private:
  std::mutex mu_;
  std::vector<std::pair<std::size_t, std::unique_ptr<quiver::ThreadPool>>> pools_;
};

/// The Filter an allowed-label array becomes. A bitset over [0, largest label] answers a lookup
/// with one word read; a hash set costs about 16 bytes per label. The bitset is chosen while its
/// words (largest / 64) stay within 16 per label plus 1024 and the largest label is below 2^32,
/// the rule python/quiver_ext.cc:40-51 applies, so both builds pick the same filter type.
std::unique_ptr<quiver::Filter> allowed_filter(const LabelArray& allowed) {
  const std::size_t count = static_cast<std::size_t>(allowed.size());
  const std::uint64_t* first = allowed.data();
  const std::uint64_t* last = first + count;
  std::uint64_t largest = 0;
  for (const std::uint64_t* it = first; it != last; ++it) largest = std::max(largest, *it);
  const bool fits_u32 = largest >> 32 == 0;
  const bool bitset_small = largest / 64 <= 16 * static_cast<std::uint64_t>(count) + 1024;
  if (!(fits_u32 && bitset_small)) return std::make_unique<quiver::LabelSetFilter>(first, last);
  auto bits = std::make_unique<quiver::BitsetFilter>(static_cast<std::size_t>(largest) + 1);
  for (const std::uint64_t* it = first; it != last; ++it) bits->insert(*it);
  return bits;
}

void check_matrix(const FloatMatrix& x, std::size_t dim) {
  if (x.ndim() != 2) throw py::value_error("expected a 2-D float32 array");
  if (static_cast<std::size_t>(x.shape(1)) != dim) {
    throw py::value_error("expected vectors of dimension " + std::to_string(dim) + ", got " +
                          std::to_string(x.shape(1)));
  }
}

/// The two result arrays of a search, allocated as numpy arrays before the search runs so the C++
/// call writes straight into them: labels int64 [nq, k] (written as quiver::Label, whose empty
/// value 2^64 - 1 reads back as -1) and distances float32 [nq, k]. More than 2^40 result slots,
/// or an nq * k that overflows, is refused with the reference's message
/// (python/quiver_ext.cc:62-68).
struct SearchResults {
  py::array_t<std::int64_t> labels;
  py::array_t<float> distances;

  SearchResults(std::size_t nq, std::size_t k) {
    std::size_t slots = 0;
    if (__builtin_mul_overflow(nq, k, &slots) || slots > (std::size_t{1} << 40)) {
      throw py::value_error("nq * k is too large");
    }
    const std::vector<py::ssize_t> shape{static_cast<py::ssize_t>(nq), static_cast<py::ssize_t>(k)};
    labels = py::array_t<std::int64_t>(shape);
    distances = py::array_t<float>(shape);
  }

  quiver::Label* label_data() { return reinterpret_cast<quiver::Label*>(labels.mutable_data()); }
  float* distance_data() { return distances.mutable_data(); }
  py::tuple as_tuple() const { return py::make_tuple(labels, distances); }
};

const std::uint64_t* optional_labels(const py::object& labels, std::size_t n, LabelArray& hold) {
  if (labels.is_none()) return nullptr;
  hold = labels.cast<LabelArray>();
  if (static_cast<std::size_t>(hold.size()) != n) {
    throw py::value_error("labels and vectors differ in length");
  }
  return hold.data();
}

}  // namespace

PYBIND11_MODULE(_quiver, m) {
  m.doc() = "Quiver search path on MI355X (gfx950): flat exact and IVF-PQ search";

  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const quiver::Error& e) {
      PyErr_SetString(PyExc_ValueError, e.what());
    }
  });

  m.def("_device_index", [] {
    int d = 0;
    if (qvh_get_device(&d) != QVH_OK) throw quiver::Error(std::string("no device: ") + qvh_last_error());
    return d;
  });

  m.def(
      "simd_isa",
      [] {
        char name[128] = {0}, arch[64] = {0};
        int cus = 0;
        if (qvh_device_info(name, sizeof(name), arch, sizeof(arch), &cus) != QVH_OK) {
          throw quiver::Error(std::string("no device: ") + qvh_last_error());
        }
        std::string a(arch);
        return a.substr(0, a.find(':'));
      },
      "Instruction set the distance kernels run on (the GPU target, e.g. gfx950).");

  py::class_<quiver::FlatIndex>(m, "FlatIndex")
      .def(py::init([](std::size_t dim, const std::string& metric) {
             return new quiver::FlatIndex(dim, quiver::parse_metric(metric));
           }),
           py::arg("dim"), py::arg("metric") = "l2")
      .def(
          "_add",
          [](quiver::FlatIndex& self, const FloatMatrix& x, const py::object& labels) {
            check_matrix(x, self.dim());
            LabelArray hold;
            const std::uint64_t* lp = optional_labels(labels, x.shape(0), hold);
            py::gil_scoped_release release;
            self.add(x.data(), x.shape(0), lp);
          },
          py::arg("vectors"), py::arg("labels").none(true))
      .def(
          "_search",
          [](const quiver::FlatIndex& self, const FloatMatrix& q, std::size_t k,
             const py::object& allowed, std::size_t threads) {
            check_matrix(q, self.dim());
            std::unique_ptr<quiver::Filter> filter;
            if (!allowed.is_none()) filter = allowed_filter(allowed.cast<LabelArray>());
            const std::size_t nq = q.shape(0);
            SearchResults out(nq, k);
            quiver::Label* labels = out.label_data();
            float* dist = out.distance_data();
            quiver::ThreadPool* pool = PoolRegistry::get(threads);
            {
              py::gil_scoped_release release;
              self.search_batch(q.data(), nq, k, labels, dist, filter.get(), pool);
            }
            return out.as_tuple();
          },
          py::arg("queries"), py::arg("k"), py::arg("allowed").none(true), py::arg("num_threads"))
      .def("save", &quiver::FlatIndex::save, py::arg("path"), py::call_guard<py::gil_scoped_release>())
      .def_static(
          "load",
          [](const std::string& path, bool verify_checksums) {
            quiver::LoadOptions o;
            o.verify_checksums = verify_checksums;
            py::gil_scoped_release release;
            return quiver::FlatIndex::load(path, o);
          },
          py::arg("path"), py::arg("verify_checksums") = true)
      .def("__len__", &quiver::FlatIndex::size, py::call_guard<py::gil_scoped_release>())
      .def("get_vector",
           [](const quiver::FlatIndex& self, std::size_t i) {
             if (i >= self.size()) throw py::index_error("row out of range");
             py::array_t<float> out(self.dim());
             std::memcpy(out.mutable_data(), self.vector(i), self.dim() * sizeof(float));
             return out;
           })
      .def_property_readonly("_device_handle",
                             [](const quiver::FlatIndex& s) { return reinterpret_cast<std::uintptr_t>(s.device_handle()); })
      .def(
          "_search_device",
          [](const quiver::FlatIndex& self, std::uintptr_t q, std::size_t nq, std::size_t k, std::uintptr_t bitmap,
             std::uintptr_t rows, std::uintptr_t dist, std::uintptr_t stream) {
            py::gil_scoped_release release;
            self.search_batch_device(reinterpret_cast<const float*>(q), nq, k,
                                     reinterpret_cast<const std::uint64_t*>(bitmap),
                                     reinterpret_cast<std::uint32_t*>(rows), reinterpret_cast<float*>(dist),
                                     reinterpret_cast<void*>(stream));
          },
          py::arg("queries"), py::arg("nq"), py::arg("k"), py::arg("bitmap"), py::arg("rows"), py::arg("distances"),
          py::arg("stream"))
      .def(
          "_search_device_rows",
          [](const quiver::FlatIndex& self, std::uintptr_t q, std::size_t nq, std::size_t k, std::uintptr_t row_list,
             std::size_t nrows, std::uintptr_t rows, std::uintptr_t dist, std::uintptr_t stream) {
            py::gil_scoped_release release;
            self.search_batch_device_rows(reinterpret_cast<const float*>(q), nq, k,
                                          reinterpret_cast<const std::uint32_t*>(row_list), nrows,
                                          reinterpret_cast<std::uint32_t*>(rows), reinterpret_cast<float*>(dist),
                                          reinterpret_cast<void*>(stream));
          },
          py::arg("queries"), py::arg("nq"), py::arg("k"), py::arg("row_list"), py::arg("nrows"), py::arg("rows"),
          py::arg("distances"), py::arg("stream"))
      .def("_row_bitmap",
           [](const quiver::FlatIndex& self, const LabelArray& allowed) {
             const auto filter = allowed_filter(allowed);
             std::vector<std::uint64_t> bits;
             {
               py::gil_scoped_release release;
               bits = self.row_bitmap(*filter);
             }
             return py::array_t<std::uint64_t>(static_cast<py::ssize_t>(bits.size()), bits.data());
           })
      .def("_labels",
           [](const quiver::FlatIndex& self) {
             const auto l = self.labels();
             return py::array_t<std::uint64_t>(static_cast<py::ssize_t>(l.size()), l.data());
           })
      .def_property_readonly("dim", &quiver::FlatIndex::dim)
      .def_property_readonly("metric", [](const quiver::FlatIndex& s) {
        return std::string(quiver::to_string(s.metric()));
      });
  py::class_<quiver::IvfPqIndex>(m, "IvfPqIndex")
      .def(py::init([](std::size_t dim, const std::string& metric, std::size_t nlist, std::size_t pq_m,
                       bool store_vectors, std::size_t train_iterations, std::uint64_t seed) {
             quiver::IvfPqParams p;
             p.dim = dim;
             p.metric = quiver::parse_metric(metric);
             p.nlist = nlist;
             p.m = pq_m;
             p.store_vectors = store_vectors;
             p.train_iterations = train_iterations;
             p.seed = seed;
             return new quiver::IvfPqIndex(p);
           }),
           py::arg("dim"), py::arg("metric") = "l2", py::arg("nlist") = 1024, py::arg("m") = 16,
           py::arg("store_vectors") = false, py::arg("train_iterations") = 20, py::arg("seed") = 1234)
      .def(
          "_train",
          [](quiver::IvfPqIndex& self, const FloatMatrix& x, std::size_t threads) {
            check_matrix(x, self.dim());
            quiver::ThreadPool* pool = PoolRegistry::get(threads);
            py::gil_scoped_release release;
            self.train(x.data(), x.shape(0), pool);
          },
          py::arg("vectors"), py::arg("num_threads"))
      .def(
          "_add",
          [](quiver::IvfPqIndex& self, const FloatMatrix& x, const py::object& labels, std::size_t threads) {
            check_matrix(x, self.dim());
            LabelArray hold;
            const std::uint64_t* lp = optional_labels(labels, x.shape(0), hold);
            quiver::ThreadPool* pool = PoolRegistry::get(threads);
            py::gil_scoped_release release;
            self.add(x.data(), x.shape(0), lp, pool);
          },
          py::arg("vectors"), py::arg("labels").none(true), py::arg("num_threads"))
      .def(
          "_search",
          [](const quiver::IvfPqIndex& self, const FloatMatrix& q, std::size_t k, std::size_t nprobe,
             std::size_t refine_factor, const py::object& allowed, std::size_t threads) {
            check_matrix(q, self.dim());
            std::unique_ptr<quiver::Filter> filter;
            if (!allowed.is_none()) filter = allowed_filter(allowed.cast<LabelArray>());
            const std::size_t nq = q.shape(0);
            SearchResults out(nq, k);
            quiver::Label* labels = out.label_data();
            float* dist = out.distance_data();
            quiver::IvfPqSearchParams p;
            p.nprobe = nprobe;
            p.refine_factor = refine_factor;
            p.filter = filter.get();
            quiver::ThreadPool* pool = PoolRegistry::get(threads);
            {
              py::gil_scoped_release release;
              self.search_batch(q.data(), nq, k, labels, dist, p, pool);
            }
            return out.as_tuple();
          },
          py::arg("queries"), py::arg("k"), py::arg("nprobe"), py::arg("refine_factor"),
          py::arg("allowed").none(true), py::arg("num_threads"))
      .def("save", &quiver::IvfPqIndex::save, py::arg("path"), py::call_guard<py::gil_scoped_release>())
      .def_static(
          "load",
          [](const std::string& path, bool verify_checksums) {
            quiver::LoadOptions o;
            o.verify_checksums = verify_checksums;
            py::gil_scoped_release release;
            return quiver::IvfPqIndex::load(path, o);
          },
          py::arg("path"), py::arg("verify_checksums") = true)
      .def("__len__", &quiver::IvfPqIndex::size, py::call_guard<py::gil_scoped_release>())
      .def_property_readonly("is_trained", &quiver::IvfPqIndex::is_trained)
      .def_property_readonly("_device_handle",
                             [](const quiver::IvfPqIndex& s) { return reinterpret_cast<std::uintptr_t>(s.device_handle()); })
      .def(
          "_search_device",
          [](const quiver::IvfPqIndex& self, std::uintptr_t q, std::size_t nq, std::size_t k, std::size_t nprobe,
             std::uint64_t refine_factor, std::uintptr_t bitmap, std::uintptr_t refs, std::uintptr_t dist,
             std::uintptr_t stream) {
            quiver::IvfPqSearchParams p;
            p.nprobe = nprobe;
            p.refine_factor = refine_factor;
            py::gil_scoped_release release;
            self.search_batch_device(reinterpret_cast<const float*>(q), nq, k, p,
                                     reinterpret_cast<const std::uint64_t*>(bitmap),
                                     reinterpret_cast<std::uint64_t*>(refs), reinterpret_cast<float*>(dist),
                                     reinterpret_cast<void*>(stream));
          },
          py::arg("queries"), py::arg("nq"), py::arg("k"), py::arg("nprobe"), py::arg("refine_factor"),
          py::arg("bitmap"), py::arg("refs"), py::arg("distances"), py::arg("stream"))
      .def("_position_bitmap",
           [](const quiver::IvfPqIndex& self, const LabelArray& allowed) {
             const auto filter = allowed_filter(allowed);
             std::vector<std::uint64_t> bits;
             {
               py::gil_scoped_release release;
               bits = self.position_bitmap(*filter);
             }
             return py::array_t<std::uint64_t>(static_cast<py::ssize_t>(bits.size()), bits.data());
           })
      .def_property_readonly("dim", &quiver::IvfPqIndex::dim)
      .def_property_readonly("nlist", [](const quiver::IvfPqIndex& s) { return s.params().nlist; })
      .def_property_readonly("m", [](const quiver::IvfPqIndex& s) { return s.params().m; })
      .def_property_readonly("metric", [](const quiver::IvfPqIndex& s) {
        return std::string(quiver::to_string(s.params().metric));
      })
      .def_property_readonly("memory_bytes",
                             [](const quiver::IvfPqIndex& s) {
                               py::gil_scoped_release release;
                               return s.memory_bytes();
                             })
      .def("list_sizes", &quiver::IvfPqIndex::list_sizes, py::call_guard<py::gil_scoped_release>())
      .def("_centroids",
           [](const quiver::IvfPqIndex& s) {
             const auto c = s.centroids();
             py::array_t<float> out({s.params().nlist, s.params().dim});
             std::memcpy(out.mutable_data(), c.data(), c.size() * sizeof(float));
             return out;
           })
      .def("_codebook",
           [](const quiver::IvfPqIndex& s) {
             const auto c = s.codebook();
             const std::size_t m = s.params().m;
             py::array_t<float> out({m, std::size_t{256}, s.params().dim / m});
             std::memcpy(out.mutable_data(), c.data(), c.size() * sizeof(float));
             return out;
           })
      .def("_set_trained",
           [](quiver::IvfPqIndex& s, const py::array_t<float, py::array::c_style>& cent,
              const py::array_t<float, py::array::c_style>& cb) {
             const auto& p = s.params();
             if (static_cast<std::size_t>(cent.size()) != p.nlist * p.dim ||
                 static_cast<std::size_t>(cb.size()) != p.m * 256 * (p.dim / p.m)) {
               throw py::value_error("trained state has the wrong size");
             }
             py::gil_scoped_release release;
             s.set_trained(cent.data(), cb.data());
           })
      .def("_list_offsets",
           [](const quiver::IvfPqIndex& s) {
             const auto v = s.list_offsets();
             py::array_t<std::uint64_t> out(v.size());
             std::memcpy(out.mutable_data(), v.data(), v.size() * sizeof(std::uint64_t));
             return out;
           })
      .def("_list_labels",
           [](const quiver::IvfPqIndex& s) {
             const auto v = s.list_labels();
             py::array_t<std::uint64_t> out(v.size());
             std::memcpy(out.mutable_data(), v.data(), v.size() * sizeof(std::uint64_t));
             return out;
           })
      .def("_list_codes",
           [](const quiver::IvfPqIndex& s) {
             std::vector<std::uint8_t> v;
             {
               py::gil_scoped_release release;
               v = s.list_codes();
             }
             const std::size_t m = s.params().m;
             py::array_t<std::uint8_t> out({v.size() / m, m});
             std::memcpy(out.mutable_data(), v.data(), v.size());
             return out;
           })
      .def("_list_vectors", [](const quiver::IvfPqIndex& s) {
        std::vector<float> v;
        {
          py::gil_scoped_release release;
          v = s.list_vectors();
        }
        const std::size_t d = s.params().dim;
        py::array_t<float> out({v.size() / d, d});
        std::memcpy(out.mutable_data(), v.data(), v.size() * sizeof(float));
        return out;
      });

  m.def(
      "kmeans",
      [](const FloatMatrix& x, std::size_t k, std::size_t iterations, std::size_t max_points_per_centroid,
         std::uint64_t seed, std::size_t threads) {
        if (x.ndim() != 2) throw py::value_error("expected a 2-D float32 array");
        quiver::KMeansParams kp;
        kp.k = k;
        kp.iterations = iterations;
        kp.max_points_per_centroid = max_points_per_centroid;
        kp.seed = seed;
        std::vector<float> c;
        const std::size_t n = x.shape(0), d = x.shape(1);
        quiver::ThreadPool* pool = PoolRegistry::get(threads);
        {
          py::gil_scoped_release release;
          c = quiver::kmeans(x.data(), n, d, kp, pool);
        }
        py::array_t<float> out({k, d});
        std::memcpy(out.mutable_data(), c.data(), c.size() * sizeof(float));
        return out;
      },
      py::arg("vectors"), py::arg("k"), py::arg("iterations") = 25, py::arg("max_points_per_centroid") = 256,
      py::arg("seed") = 1234, py::arg("num_threads") = 0,
      "Lloyd's k-means (the reference's kmeans), assignment steps on the GPU.");
}
