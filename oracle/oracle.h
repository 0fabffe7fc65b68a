/*
 * ORACLE — test infrastructure, NOT product code.
 *
 * A plain-C restatement of the CPU algorithms of TheWiseGhost/quiver's data-parallel search path
 * (flat exact search, IVF-PQ train / add / search, PQ encode, k-means). Only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it, and only to check the
 * device's results (or, in the bench, as the timed CPU baseline). The product (quiver_amd) never
 * links or calls it.
 *
 * Every function cites the reference file:line it restates. Floating-point operations follow the
 * reference's exact order and rounding: the file is compiled with -ffp-contract=off; the AVX2
 * kernels' fused multiply-adds are written as fmaf().
 *
 * Deliberate difference: where the reference's result order among EXACTLY equal distances is an
 * artifact of libstdc++ heap mechanics (dist-only comparators, src/internal/search_util.h:26-28;
 * std::partial_sort of probes, src/ivfpq_index.cc:298-300), the oracle uses the deterministic
 * lexicographic order (distance, id). Comparisons against the reference's golden vectors are
 * therefore tie-aware (see tests/parity.py).
 *
 * Pinning: each function is checked in tests/test_oracle_golden.py against golden vectors made by
 * the compiled reference (tests/golden/), against the C++ standard's known answer for
 * mt19937_64, and against float64 closed forms. No function here is "parity unpinned".
 */
#ifndef QUIVER_ORACLE_H
#define QUIVER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_L2 = 0, ORC_IP = 1, ORC_COSINE = 2 };

/* mt19937_64 (std::mt19937_64, [rand.predef]) */
typedef struct {
  uint64_t mt[312];
  int idx;
} orc_mt64;
void orc_mt64_seed(orc_mt64* g, uint64_t seed);
uint64_t orc_mt64_next(orc_mt64* g);
/* std::uniform_real_distribution<double>(0,1) via libstdc++ generate_canonical<double,53>. */
double orc_mt64_canonical(orc_mt64* g);

/* Distance kernels: AVX2+FMA reduction order (src/simd/kernels_avx2.cc:35-83) and the scalar
 * kernels (src/simd/kernels_scalar.cc:7-22). The AVX2 tail (< 8 elements) follows what GCC 11
 * -O3 emits for it: the first four products separately rounded, the rest fused. */
float orc_l2sqr_avx2(const float* a, const float* b, size_t dim);
float orc_dot_avx2(const float* a, const float* b, size_t dim);
float orc_l2sqr_scalar(const float* a, const float* b, size_t dim);
float orc_dot_scalar(const float* a, const float* b, size_t dim);
/* simd::normalize (src/simd/dispatch.cc:119-135) with the AVX2 dot; n rows in place. */
void orc_normalize(float* v, size_t n, size_t dim);

/* CentroidTable arithmetic (src/internal/centroid_table.h). Centroids are row-major k x dim. */
void orc_ct_l2(const float* x, const float* cent, size_t k, size_t dim, float* out);
void orc_ct_dot(const float* x, const float* cent, size_t k, size_t dim, float* out);
size_t orc_argmin_n(const float* v, size_t n);
/* nearest_centroid, src/product_quantizer.cc:14-27 */
size_t orc_nearest_centroid(const float* x, const float* centroids, size_t k, size_t dim);
void orc_nearest_batch(const float* x, size_t n, const float* cent, size_t k, size_t dim,
                       int max_inner_product, uint32_t* out, int nthreads);

/* FlatIndex::search_batch (src/flat_index.cc:69-107,126-140) over stored rows. Queries are
 * normalized here for cosine (as search_one does); rows must already be stored normalized.
 * row_bitmap: NULL or ceil(n/64) words, bit i = row i admitted. Outputs nq*k rows (UINT32_MAX =
 * empty) and distances (+inf = empty), ascending (distance, row). */
int orc_flat_search(const float* base, size_t n, size_t dim, int metric, const float* queries,
                    size_t nq, size_t k, const uint64_t* row_bitmap, int nthreads,
                    uint32_t* out_rows, float* out_dist);
/* The flat distance of (query i, row r) pairs, exactly as search_one computes it. */
void orc_flat_pair_dist(const float* base, size_t dim, int metric, const float* queries,
                        size_t npairs, const uint64_t* qidx, const uint64_t* ridx, float* out);

/* kmeans (src/product_quantizer.cc:29-117). out: k x dim. */
int orc_kmeans(const float* x, size_t n, size_t dim, size_t k, size_t iterations,
               size_t max_points_per_centroid, uint64_t seed, int nthreads, float* out);
/* ProductQuantizer::train (src/product_quantizer.cc:133-153). codebook: m x 256 x dsub. */
int orc_pq_train(const float* x, size_t n, size_t dim, size_t m, size_t iterations, uint64_t seed,
                 int nthreads, float* codebook);
/* ProductQuantizer::encode (src/product_quantizer.cc:165-171). */
void orc_pq_encode(const float* codebook, size_t dim, size_t m, const float* x, size_t n,
                   uint8_t* codes, int nthreads);
/* compute_l2_table / compute_ip_table (src/product_quantizer.cc:180-186). */
void orc_pq_tables(const float* codebook, size_t dim, size_t m, const float* q, float* l2_table,
                   float* ip_table);
/* adc (src/product_quantizer.cc:188-192), n codes. */
void orc_pq_adc(const float* table, size_t m, const uint8_t* codes, size_t n, float* out);

/* IVF-PQ. */
typedef struct {
  size_t dim, nlist, m;
  int metric;
  const float* centroids;   /* nlist x dim */
  const float* codebook;    /* m x 256 x dsub */
  const float* precomputed; /* nlist x m x 256, or NULL */
  const uint64_t* offsets;  /* nlist + 1 (CSR over lists) */
  const uint8_t* codes;     /* count x m, list order */
  const float* vectors;     /* count x dim or NULL (store_vectors) */
} orc_ivfpq;

/* Impl::train (src/ivfpq_index.cc:144-206). Writes centroids (nlist x dim), codebook, and the
 * precomputed table (nlist x m x 256) when `precomputed` is non-NULL and it applies; returns 1 if
 * a precomputed table was written, 0 if not, <0 on error. */
int orc_ivfpq_train(const float* x, size_t n, size_t dim, int metric, size_t nlist, size_t m,
                    size_t iterations, uint64_t seed, int nthreads, float* centroids,
                    float* codebook, float* precomputed);
/* Impl::precompute (src/ivfpq_index.cc:112-129). */
void orc_ivfpq_precompute(const float* centroids, const float* codebook, size_t nlist, size_t dim,
                          size_t m, float* out);
/* Impl::add's encode step (src/ivfpq_index.cc:208-246): cell and code of each vector. For
 * cosine, `x` is normalized first into `x_stored` (may be NULL otherwise). */
void orc_ivfpq_encode(const float* centroids, const float* codebook, size_t nlist, size_t dim,
                      size_t m, int metric, const float* x, size_t n, int nthreads,
                      uint32_t* assign, uint8_t* codes, float* x_stored);
/* Impl::search_into (src/ivfpq_index.cc:275-381). pos_bitmap: NULL or a bitmap over CSR
 * positions (admitted vectors). out_refs: (list << 32) | offset, UINT64_MAX = empty. */
int orc_ivfpq_search(const orc_ivfpq* ix, const float* queries, size_t nq, size_t k,
                     size_t nprobe, size_t refine_factor, const uint64_t* pos_bitmap,
                     int nthreads, uint64_t* out_refs, float* out_dist);
/* Per-query coarse scores (L2: ||q-c||^2 sequential; IP/cosine: -<q,c>) and the first nprobe
 * lists by (score, list). For checking the device's probe selection. */
#ifdef __cplusplus
}
#endif
#endif
