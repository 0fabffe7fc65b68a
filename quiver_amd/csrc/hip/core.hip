// Process-wide state of the qvh library: error reporting, device selection, the allocation
// fault hook, and row normalization.
#include <atomic>
#include <cstdlib>
#include <string>

#include "common.hpp"
#include "exact.hpp"

namespace qvh {
namespace {

thread_local std::string t_last_error;

std::mutex g_device_mu;
int g_device = -1;     // device chosen by qvh_init (or 0 on first use)
bool g_checked = false;

std::atomic<long> g_alloc_count{0};
long fault_alloc_at() {
  static const long at = [] {
    const char* s = std::getenv("QVH_FAULT_ALLOC");
    return s && *s ? std::atol(s) : 0L;
  }();
  return at;
}

void check_device(int dev) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    throw Failure(QVH_EDEVICE, "no HIP device is available (the qvh kernels need a gfx950 GPU)");
  }
  if (dev < 0 || dev >= count) {
    throw Failure(QVH_EINVAL, "device " + std::to_string(dev) + " does not exist (" +
                                  std::to_string(count) + " HIP devices)");
  }
  hipDeviceProp_t prop;
  QVH_HIP(hipGetDeviceProperties(&prop, dev));
  if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) {
    throw Failure(QVH_EDEVICE, std::string("device is ") + prop.gcnArchName +
                                   "; the qvh kernels are built for gfx950 only");
  }
}

// simd::normalize (src/simd/dispatch.cc:119-135) of every row in place, eight lanes per row: the
// group computes the row's dot product in the reference's order (exact_group8, bit for bit as
// exact_dot), every lane then scales its share of the row by the same 1/sqrt(norm^2). A non-finite
// sum takes the double-precision redo in the group's first lane, as exact_normalize does.
__global__ void normalize_rows_kernel(float* __restrict__ rows, uint64_t n, uint32_t dim) {
  const uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t r = t >> 3;
  const uint32_t l = static_cast<uint32_t>(t & 7u);
  const bool valid = r < n;
  float* v = rows + (valid ? r : 0) * dim;
  const float lead = exact_group8<false>(v, v, dim, valid);  // every lane of the wave takes part
  const float norm_sq = __shfl(lead, 0, 8);
  if (!valid) return;
  if (!isfinite(norm_sq)) {
    if (l == 0) exact_normalize(v, dim);
    return;
  }
  if (norm_sq <= 0.0f) return;
  const float inv = 1.0f / sqrtf(norm_sq);
  for (uint32_t i = l; i < dim; i += 8) v[i] = v[i] * inv;
}

}  // namespace

void set_last_error(const std::string& msg) { t_last_error = msg; }

int current_device() {
  std::lock_guard<std::mutex> lock(g_device_mu);
  if (g_device < 0) g_device = 0;
  if (!g_checked) {
    check_device(g_device);
    g_checked = true;
  }
  QVH_HIP(hipSetDevice(g_device));
  return g_device;
}

void* device_alloc(size_t bytes) {
  const long n = ++g_alloc_count;
  if (fault_alloc_at() > 0 && n == fault_alloc_at()) {
    throw Failure(QVH_ENOMEM, "injected allocation failure (QVH_FAULT_ALLOC=" +
                                  std::to_string(n) + ")");
  }
  void* p = nullptr;
  QVH_HIP(hipMalloc(&p, bytes == 0 ? 1 : bytes));
  return p;
}

void device_free(void* p) noexcept {
  // Asynchronous work of any stream may still read a buffer that is regrown or released: the
  // device finishes it first.
  if (p) {
    (void)hipDeviceSynchronize();
    (void)hipFree(p);
  }
}

void launch_normalize_rows(float* d_rows, uint64_t n, uint32_t dim, hipStream_t stream) {
  if (n == 0) return;
  const unsigned block = 256;  // 32 rows
  hipLaunchKernelGGL(normalize_rows_kernel, dim3(static_cast<unsigned>(ceil_div(n * 8, block))),
                     dim3(block), 0, stream, d_rows, n, dim);
  QVH_HIP(hipGetLastError());
}

}  // namespace qvh

extern "C" {

const char* qvh_last_error(void) { return qvh::t_last_error.c_str(); }

qvh_status qvh_device_allocations(uint64_t* count) {
  if (count == nullptr) {
    qvh::set_last_error("qvh_device_allocations: null output");
    return QVH_EINVAL;
  }
  *count = static_cast<uint64_t>(qvh::g_alloc_count.load());
  return QVH_OK;
}

qvh_status qvh_init(int device) {
  return qvh::guarded([&] {
    std::lock_guard<std::mutex> lock(qvh::g_device_mu);
    qvh::check_device(device);
    qvh::g_device = device;
    qvh::g_checked = true;
    QVH_HIP(hipSetDevice(device));
  });
}

qvh_status qvh_get_device(int* device) {
  return qvh::guarded([&] {
    QVH_REQUIRE(device != nullptr, "qvh_get_device: null argument");
    *device = qvh::current_device();
  });
}

qvh_status qvh_device_info(char* name, size_t name_len, char* arch, size_t arch_len,
                           int* compute_units) {
  return qvh::guarded([&] {
    const int dev = qvh::current_device();
    hipDeviceProp_t prop;
    QVH_HIP(hipGetDeviceProperties(&prop, dev));
    if (name && name_len) {
      std::strncpy(name, prop.name, name_len - 1);
      name[name_len - 1] = '\0';
    }
    if (arch && arch_len) {
      std::strncpy(arch, prop.gcnArchName, arch_len - 1);
      arch[arch_len - 1] = '\0';
    }
    if (compute_units) *compute_units = prop.multiProcessorCount;
  });
}

qvh_status qvh_normalize(float* rows, uint64_t n, uint32_t dim) {
  return qvh::guarded([&] {
    QVH_REQUIRE(rows != nullptr || n == 0, "qvh_normalize: null rows");
    QVH_REQUIRE(dim >= 1, "qvh_normalize: dim must be positive");
    if (n == 0) return;
    qvh::current_device();
    qvh::DeviceBuffer buf;
    const size_t bytes = static_cast<size_t>(n) * dim * sizeof(float);
    float* d = static_cast<float*>(buf.reserve(bytes));
    QVH_HIP(hipMemcpy(d, rows, bytes, hipMemcpyHostToDevice));
    qvh::launch_normalize_rows(d, n, dim, nullptr);
    QVH_HIP(hipMemcpy(rows, d, bytes, hipMemcpyDeviceToHost));
  });
}

}  // extern "C"
