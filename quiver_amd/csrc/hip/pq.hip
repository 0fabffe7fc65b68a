// ProductQuantizer and nearest_centroid on gfx950 (src/product_quantizer.cc:14-27,155-217): PQ
// encode, decode, ADC tables and ADC sums over batches of vectors, and the nearest centroid of
// each of a batch of points. Every sum replays the reference's in-order float arithmetic (all qvh
// sources are compiled with -ffp-contract=off), so codes, tables, sums and indices are bit-identical.
#include <algorithm>
#include <cstring>

#include "common.hpp"
#include "exact.hpp"

namespace qvh {
void launch_pq_encode(const float* d_x, uint64_t n, uint32_t dim, uint32_t m, const float* d_cbt, uint8_t* d_codes,
                      hipStream_t s);
void launch_codebook_transpose(const float* d_cb, uint32_t m, uint32_t dsub, float* d_cbt, hipStream_t s);
}  // namespace qvh

namespace {

using namespace qvh;

/// ProductQuantizer::decode (src/product_quantizer.cc:173-178): out[i][j * dsub + t] =
/// codebook[j][code_ij][t]. One thread per output value.
__global__ void pq_decode_kernel(const float* __restrict__ cb, const uint8_t* __restrict__ codes, uint64_t n,
                                 uint32_t m, uint32_t dsub, float* __restrict__ out) {
  const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint32_t dim = m * dsub;
  if (e >= n * dim) return;
  const uint64_t i = e / dim;
  const uint32_t f = static_cast<uint32_t>(e % dim), j = f / dsub, t = f % dsub;
  out[e] = cb[(static_cast<uint64_t>(j) * 256 + codes[i * m + j]) * dsub + t];
}

/// compute_l2_table / compute_ip_table (src/product_quantizer.cc:180-186 over CentroidTable::l2 /
/// dot, src/internal/centroid_table.h:65-85): table[q][j][c] = sum_t (q_t - c_t)^2 or
/// sum_t q_t * c_t over the sub-vector, in order of t. One thread per entry; consecutive threads
/// read consecutive codewords of the transposed codebook.
__global__ void pq_tables_kernel(const float* __restrict__ Q, uint64_t nq, uint32_t m, uint32_t dsub,
                                 const float* __restrict__ cbt, int inner_product, float* __restrict__ out) {
  const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= nq * m * 256) return;
  const uint32_t c = e % 256, j = (e / 256) % m;
  const uint64_t q = e / (256ull * m);
  const float* qj = Q + q * m * dsub + static_cast<uint64_t>(j) * dsub;
  const float* col = cbt + static_cast<uint64_t>(j) * dsub * 256 + c;
  float v = 0.0f;
  for (uint32_t t = 0; t < dsub; ++t) {
    if (inner_product) {
      v = v + qj[t] * col[t * 256];
    } else {
      const float d = qj[t] - col[t * 256];
      v = v + d * d;
    }
  }
  out[e] = v;
}

/// ProductQuantizer::adc / adc_batch (src/product_quantizer.cc:188-217): sum_j table[j][code_j] in
/// order of j (adc_batch's four interleaved chains are four such sums). One thread per code.
__global__ void pq_adc_kernel(const float* __restrict__ table, const uint8_t* __restrict__ codes, uint64_t n,
                              uint32_t m, float* __restrict__ out) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint8_t* c = codes + i * m;
  float s = 0.0f;
  for (uint32_t j = 0; j < m; ++j) s = s + table[j * 256 + c[j]];
  out[i] = s;
}

/// nearest_centroid (src/product_quantizer.cc:14-27): the first c with the smallest
/// simd::l2sqr(x, centroid_c) among the distances below +inf (strict <, starting from +inf), 0 if
/// there is none. One block per point; each thread takes centroids tid, tid + 256, ... with the
/// reference's AVX2 reduction order, then the block takes the smallest (distance, index) key.
__global__ void __launch_bounds__(256) nearest_centroid_kernel(const float* __restrict__ x, uint64_t n,
                                                               const float* __restrict__ cent, uint32_t k,
                                                               uint32_t dim, uint32_t* __restrict__ out) {
  __shared__ uint64_t s_best[4];
  const uint64_t p = blockIdx.x;
  const float* xp = x + p * dim;
  uint64_t best = ~0ull;
  for (uint32_t c = threadIdx.x; c < k; c += 256) {
    const float d = exact_l2sqr(xp, cent + static_cast<uint64_t>(c) * dim, dim);
    if (d < __builtin_huge_valf()) {  // NaN and +inf never win (d < best_d fails for them)
      const uint64_t key = make_key(d, c);
      best = key < best ? key : best;
    }
  }
  best = wave_min_u64(best);
  if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = s_best[0];
    for (int w = 1; w < 4; ++w) b = s_best[w] < b ? s_best[w] : b;
    out[p] = b == ~0ull ? 0u : static_cast<uint32_t>(b);
  }
}

}  // namespace

struct qvh_pq {
  uint32_t dim = 0, m = 0, dsub = 0;
  int device = 0;
  DeviceBuffer cb, cbt;   // [m][256][dsub] and per sub-space transposed [m][dsub][256]
  DeviceBuffer w_in, w_out, w_codes, w_table;
  hipStream_t stream = nullptr;
  std::mutex mu;
};

extern "C" {

qvh_status qvh_pq_create(uint32_t dim, uint32_t m, const float* codebook, qvh_pq** out) {
  return guarded([&] {
    QVH_REQUIRE(out != nullptr, "qvh_pq_create: null output");
    *out = nullptr;
    QVH_REQUIRE(codebook != nullptr, "qvh_pq_create: null codebook");
    QVH_REQUIRE(dim >= 1 && m >= 1 && dim % m == 0, "PQ: dimension must be divisible by m");
    const int dev = current_device();
    auto* p = new qvh_pq;
    p->dim = dim;
    p->m = m;
    p->dsub = dim / m;
    p->device = dev;
    const hipError_t e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete p;
      throw Failure(QVH_EDEVICE, std::string("hipStreamCreate: ") + hipGetErrorString(e));
    }
    try {
      const size_t bytes = static_cast<size_t>(m) * 256 * p->dsub * sizeof(float);
      p->cb.reserve(bytes);
      p->cbt.reserve(bytes);
      QVH_HIP(hipMemcpyAsync(p->cb.ptr, codebook, bytes, hipMemcpyHostToDevice, p->stream));
      launch_codebook_transpose(p->cb.as<float>(), m, p->dsub, p->cbt.as<float>(), p->stream);
      QVH_HIP(hipStreamSynchronize(p->stream));
    } catch (...) {
      qvh_pq_destroy(p);
      throw;
    }
    *out = p;
  });
}

void qvh_pq_destroy(qvh_pq* p) {
  if (!p) return;
  (void)hipSetDevice(p->device);
  if (p->stream) {
    (void)hipStreamSynchronize(p->stream);
    (void)hipStreamDestroy(p->stream);
  }
  delete p;
}

qvh_status qvh_pq_encode(qvh_pq* p, const float* x, uint64_t n, uint8_t* codes) {
  return guarded([&] {
    QVH_REQUIRE(p != nullptr, "qvh_pq_encode: null handle");
    if (n == 0) return;
    QVH_REQUIRE(x && codes, "qvh_pq_encode: null buffer");
    std::lock_guard<std::mutex> lock(p->mu);
    QVH_HIP(hipSetDevice(p->device));
    const size_t xb = n * p->dim * sizeof(float);
    float* dx = static_cast<float*>(p->w_in.reserve(xb));
    uint8_t* dc = static_cast<uint8_t*>(p->w_codes.reserve(n * p->m));
    QVH_HIP(hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, p->stream));
    launch_pq_encode(dx, n, p->dim, p->m, p->cbt.as<float>(), dc, p->stream);
    QVH_HIP(hipMemcpyAsync(codes, dc, n * p->m, hipMemcpyDeviceToHost, p->stream));
    QVH_HIP(hipStreamSynchronize(p->stream));
  });
}

qvh_status qvh_pq_decode(qvh_pq* p, const uint8_t* codes, uint64_t n, float* out) {
  return guarded([&] {
    QVH_REQUIRE(p != nullptr, "qvh_pq_decode: null handle");
    if (n == 0) return;
    QVH_REQUIRE(codes && out, "qvh_pq_decode: null buffer");
    std::lock_guard<std::mutex> lock(p->mu);
    QVH_HIP(hipSetDevice(p->device));
    uint8_t* dc = static_cast<uint8_t*>(p->w_codes.reserve(n * p->m));
    const size_t ob = n * p->dim * sizeof(float);
    float* dout = static_cast<float*>(p->w_out.reserve(ob));
    QVH_HIP(hipMemcpyAsync(dc, codes, n * p->m, hipMemcpyHostToDevice, p->stream));
    hipLaunchKernelGGL(pq_decode_kernel, dim3(static_cast<unsigned>(ceil_div(n * p->dim, 256))), dim3(256), 0,
                       p->stream, p->cb.as<float>(), dc, n, p->m, p->dsub, dout);
    QVH_HIP(hipGetLastError());
    QVH_HIP(hipMemcpyAsync(out, dout, ob, hipMemcpyDeviceToHost, p->stream));
    QVH_HIP(hipStreamSynchronize(p->stream));
  });
}

qvh_status qvh_pq_tables(qvh_pq* p, const float* queries, uint64_t nq, int inner_product, float* tables) {
  return guarded([&] {
    QVH_REQUIRE(p != nullptr, "qvh_pq_tables: null handle");
    if (nq == 0) return;
    QVH_REQUIRE(queries && tables, "qvh_pq_tables: null buffer");
    std::lock_guard<std::mutex> lock(p->mu);
    QVH_HIP(hipSetDevice(p->device));
    const size_t qb = nq * p->dim * sizeof(float);
    const uint64_t entries = nq * p->m * 256;
    float* dq = static_cast<float*>(p->w_in.reserve(qb));
    float* dt = static_cast<float*>(p->w_table.reserve(entries * sizeof(float)));
    QVH_HIP(hipMemcpyAsync(dq, queries, qb, hipMemcpyHostToDevice, p->stream));
    hipLaunchKernelGGL(pq_tables_kernel, dim3(static_cast<unsigned>(ceil_div(entries, 256))), dim3(256), 0, p->stream,
                       dq, nq, p->m, p->dsub, p->cbt.as<float>(), inner_product ? 1 : 0, dt);
    QVH_HIP(hipGetLastError());
    QVH_HIP(hipMemcpyAsync(tables, dt, entries * sizeof(float), hipMemcpyDeviceToHost, p->stream));
    QVH_HIP(hipStreamSynchronize(p->stream));
  });
}

qvh_status qvh_pq_adc(qvh_pq* p, const float* table, const uint8_t* codes, uint64_t n, float* out) {
  return guarded([&] {
    QVH_REQUIRE(p != nullptr, "qvh_pq_adc: null handle");
    if (n == 0) return;
    QVH_REQUIRE(table && codes && out, "qvh_pq_adc: null buffer");
    std::lock_guard<std::mutex> lock(p->mu);
    QVH_HIP(hipSetDevice(p->device));
    const size_t tb = static_cast<size_t>(p->m) * 256 * sizeof(float);
    float* dt = static_cast<float*>(p->w_table.reserve(tb));
    uint8_t* dc = static_cast<uint8_t*>(p->w_codes.reserve(n * p->m));
    float* dout = static_cast<float*>(p->w_out.reserve(n * sizeof(float)));
    QVH_HIP(hipMemcpyAsync(dt, table, tb, hipMemcpyHostToDevice, p->stream));
    QVH_HIP(hipMemcpyAsync(dc, codes, n * p->m, hipMemcpyHostToDevice, p->stream));
    hipLaunchKernelGGL(pq_adc_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, p->stream, dt, dc,
                       n, p->m, dout);
    QVH_HIP(hipGetLastError());
    QVH_HIP(hipMemcpyAsync(out, dout, n * sizeof(float), hipMemcpyDeviceToHost, p->stream));
    QVH_HIP(hipStreamSynchronize(p->stream));
  });
}

qvh_status qvh_nearest_centroid(const float* x, uint64_t n, const float* centroids, uint32_t k, uint32_t dim,
                                uint32_t* out) {
  return guarded([&] {
    if (n == 0) return;
    QVH_REQUIRE(x && centroids && out, "qvh_nearest_centroid: null buffer");
    QVH_REQUIRE(k >= 1 && dim >= 1, "qvh_nearest_centroid: k and dim must be positive");
    QVH_REQUIRE(n <= 0x7FFFFFFFull, "qvh_nearest_centroid: too many points in one call");
    current_device();
    DeviceBuffer dx, dc, dout;
    const size_t xb = n * dim * sizeof(float), cb = static_cast<size_t>(k) * dim * sizeof(float);
    dx.reserve(xb);
    dc.reserve(cb);
    dout.reserve(n * sizeof(uint32_t));
    QVH_HIP(hipMemcpy(dx.ptr, x, xb, hipMemcpyHostToDevice));
    QVH_HIP(hipMemcpy(dc.ptr, centroids, cb, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(nearest_centroid_kernel, dim3(static_cast<unsigned>(n)), dim3(256), 0, nullptr, dx.as<float>(),
                       n, dc.as<float>(), k, dim, dout.as<uint32_t>());
    QVH_HIP(hipGetLastError());
    QVH_HIP(hipMemcpy(out, dout.ptr, n * sizeof(uint32_t), hipMemcpyDeviceToHost));
  });
}

}  // extern "C"
