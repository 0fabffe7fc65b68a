/*
 * ORACLE — test infrastructure, NOT product code. See oracle.h for the contract.
 *
 * Compiled with -ffp-contract=off: every a*b+c below is two roundings unless written fmaf().
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* mt19937_64: the C++ standard's parameters ([rand.predef], std::mt19937_64). The reference's  */
/* k-means and PQ subset draw from it (src/product_quantizer.cc:36, src/ivfpq_index.cc:187).    */
/* ------------------------------------------------------------------------------------------ */
#define MT_N 312
#define MT_M 156
#define MT_UPPER 0xFFFFFFFF80000000ULL
#define MT_LOWER 0x7FFFFFFFULL

void orc_mt64_seed(orc_mt64* g, uint64_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < MT_N; ++i) {
    g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
  }
  g->idx = MT_N;
}

uint64_t orc_mt64_next(orc_mt64* g) {
  if (g->idx >= MT_N) {
    for (int i = 0; i < MT_N; ++i) {
      const uint64_t y = (g->mt[i] & MT_UPPER) | (g->mt[(i + 1) % MT_N] & MT_LOWER);
      uint64_t v = g->mt[(i + MT_M) % MT_N] ^ (y >> 1);
      if (y & 1ULL) v ^= 0xB5026F5AA96619E9ULL;
      g->mt[i] = v;
    }
    g->idx = 0;
  }
  uint64_t z = g->mt[g->idx++];
  z ^= (z >> 29) & 0x5555555555555555ULL;
  z ^= (z << 17) & 0x71D67FFFEDA60000ULL;
  z ^= (z << 37) & 0xFFF7EEE000000000ULL;
  z ^= z >> 43;
  return z;
}

/* libstdc++ generate_canonical<double, 53>(mt19937_64): one draw (the engine yields 64 bits),
 * converted to double and divided by 2^64; a result of 1.0 is replaced by nextafter(1, 0). */
double orc_mt64_canonical(orc_mt64* g) {
  const double r = (double)orc_mt64_next(g) / 18446744073709551616.0;
  return r >= 1.0 ? nextafter(1.0, 0.0) : r;
}

/* ------------------------------------------------------------------------------------------ */
/* Distance kernels                                                                            */
/* ------------------------------------------------------------------------------------------ */

/* hsum of the AVX2 kernels (src/simd/kernels_avx2.cc:17-23): lo[j] = v[j] + v[j+4], then
 * (lo0 + lo1) + (lo2 + lo3). */
static float avx2_hsum(const float v[8]) {
  float lo[4];
  for (int j = 0; j < 4; ++j) lo[j] = v[j] + v[j + 4];
  return (lo[0] + lo[1]) + (lo[2] + lo[3]);
}

/* src/simd/kernels_avx2.cc:35-56. Four 8-lane FMA accumulators over blocks of 32, an 8-wide
 * loop into s0, hsum((s0+s1)+(s2+s3)), then the scalar tail as GCC 11 -O3 compiles it inside the
 * target("avx2,fma") function. */
float orc_l2sqr_avx2(const float* a, const float* b, size_t dim) {
  float s[4][8];
  memset(s, 0, sizeof(s));
  size_t i = 0;
  for (; i + 32 <= dim; i += 32) {
    for (int u = 0; u < 4; ++u) {
      for (int l = 0; l < 8; ++l) {
        const float d = a[i + 8 * u + l] - b[i + 8 * u + l];
        s[u][l] = fmaf(d, d, s[u][l]);
      }
    }
  }
  for (; i + 8 <= dim; i += 8) {
    for (int l = 0; l < 8; ++l) {
      const float d = a[i + l] - b[i + l];
      s[0][l] = fmaf(d, d, s[0][l]);
    }
  }
  float v[8];
  for (int l = 0; l < 8; ++l) v[l] = (s[0][l] + s[1][l]) + (s[2][l] + s[3][l]);
  float sum = avx2_hsum(v);
  /* Tail (< 8 elements): GCC -O3 vectorizes the first four products (separately rounded, then
   * added in order) and contracts the remaining ones into FMAs. */
  const size_t v4 = i + (dim - i) / 4 * 4;
  for (; i < v4; ++i) {
    const float d = a[i] - b[i];
    sum += d * d;
  }
  for (; i < dim; ++i) {
    const float d = a[i] - b[i];
    sum = fmaf(d, d, sum);
  }
  return sum;
}

/* src/simd/kernels_avx2.cc:58-83. */
float orc_dot_avx2(const float* a, const float* b, size_t dim) {
  float s[4][8];
  memset(s, 0, sizeof(s));
  size_t i = 0;
  for (; i + 32 <= dim; i += 32) {
    for (int u = 0; u < 4; ++u) {
      for (int l = 0; l < 8; ++l) s[u][l] = fmaf(a[i + 8 * u + l], b[i + 8 * u + l], s[u][l]);
    }
  }
  for (; i + 8 <= dim; i += 8) {
    for (int l = 0; l < 8; ++l) s[0][l] = fmaf(a[i + l], b[i + l], s[0][l]);
  }
  float v[8];
  for (int l = 0; l < 8; ++l) v[l] = (s[0][l] + s[1][l]) + (s[2][l] + s[3][l]);
  float sum = avx2_hsum(v);
  const size_t v4 = i + (dim - i) / 4 * 4; /* tail: see orc_l2sqr_avx2 */
  for (; i < v4; ++i) sum += a[i] * b[i];
  for (; i < dim; ++i) sum = fmaf(a[i], b[i], sum);
  return sum;
}

/* src/simd/kernels_scalar.cc:7-22 */
float orc_l2sqr_scalar(const float* a, const float* b, size_t dim) {
  float sum = 0.0f;
  for (size_t i = 0; i < dim; ++i) {
    const float d = a[i] - b[i];
    sum += d * d;
  }
  return sum;
}
float orc_dot_scalar(const float* a, const float* b, size_t dim) {
  float sum = 0.0f;
  for (size_t i = 0; i < dim; ++i) sum += a[i] * b[i];
  return sum;
}

/* src/simd/dispatch.cc:119-135 */
static void normalize_one(float* v, size_t dim) {
  const float norm_sq = orc_dot_avx2(v, v, dim);
  if (!isfinite(norm_sq)) {
    double acc = 0.0;
    for (size_t i = 0; i < dim; ++i) acc += (double)v[i] * (double)v[i];
    const double inv = acc > 0.0 && isfinite(acc) ? 1.0 / sqrt(acc) : 0.0;
    if (inv == 0.0) return;
    for (size_t i = 0; i < dim; ++i) v[i] = (float)((double)v[i] * inv);
    return;
  }
  if (norm_sq <= 0.0f) return;
  const float inv = 1.0f / sqrtf(norm_sq);
  for (size_t i = 0; i < dim; ++i) v[i] *= inv;
}

void orc_normalize(float* v, size_t n, size_t dim) {
  for (size_t i = 0; i < n; ++i) normalize_one(v + i * dim, dim);
}

/* ------------------------------------------------------------------------------------------ */
/* CentroidTable (src/internal/centroid_table.h)                                               */
/* ------------------------------------------------------------------------------------------ */

static int nthreads_or_max(int nthreads) { return nthreads > 0 ? nthreads : omp_get_max_threads(); }

/* Transposed copy t[j*k + c] = cent[c*dim + j] (centroid_table.h:50-57). */
static float* transpose(const float* cent, size_t k, size_t dim) {
  float* t = (float*)malloc(sizeof(float) * k * dim);
  for (size_t c = 0; c < k; ++c)
    for (size_t j = 0; j < dim; ++j) t[j * k + c] = cent[c * dim + j];
  return t;
}

/* ||c||^2, sequential over j (centroid_table.h:50-57). */
static void ct_norms(const float* cent, size_t k, size_t dim, float* norms) {
  for (size_t c = 0; c < k; ++c) {
    float norm = 0.0f;
    for (size_t j = 0; j < dim; ++j) {
      const float v = cent[c * dim + j];
      norm += v * v;
    }
    norms[c] = norm;
  }
}

static void ct_l2_t(const float* x, const float* t, size_t k, size_t dim, float* out) {
  for (size_t c = 0; c < k; ++c) out[c] = 0.0f;
  for (size_t j = 0; j < dim; ++j) {
    const float xj = x[j];
    const float* row = t + j * k;
    for (size_t c = 0; c < k; ++c) {
      const float d = xj - row[c];
      out[c] += d * d;
    }
  }
}

static void ct_dot_t(const float* x, const float* t, size_t k, size_t dim, float* out) {
  for (size_t c = 0; c < k; ++c) out[c] = 0.0f;
  for (size_t j = 0; j < dim; ++j) {
    const float xj = x[j];
    const float* row = t + j * k;
    for (size_t c = 0; c < k; ++c) out[c] += xj * row[c];
  }
}

/* centroid_table.h:65-75 */
void orc_ct_l2(const float* x, const float* cent, size_t k, size_t dim, float* out) {
  float* t = transpose(cent, k, dim);
  ct_l2_t(x, t, k, dim, out);
  free(t);
}

/* centroid_table.h:78-85 */
void orc_ct_dot(const float* x, const float* cent, size_t k, size_t dim, float* out) {
  float* t = transpose(cent, k, dim);
  ct_dot_t(x, t, k, dim, out);
  free(t);
}

/* centroid_table.h:155-170: the min over 4 interleaved chains of std::min (NaN never wins),
 * then the first index holding that value; 0 if none does. */
size_t orc_argmin_n(const float* v, size_t n) {
  float m0 = INFINITY, m1 = INFINITY, m2 = INFINITY, m3 = INFINITY;
  size_t i = 0;
#define STDMIN(a, b) ((b) < (a) ? (b) : (a))
  for (; i + 4 <= n; i += 4) {
    m0 = STDMIN(m0, v[i]);
    m1 = STDMIN(m1, v[i + 1]);
    m2 = STDMIN(m2, v[i + 2]);
    m3 = STDMIN(m3, v[i + 3]);
  }
  for (; i < n; ++i) m0 = STDMIN(m0, v[i]);
  const float m = STDMIN(STDMIN(m0, m1), STDMIN(m2, m3));
#undef STDMIN
  for (size_t j = 0; j < n; ++j) {
    if (v[j] == m) return j;
  }
  return 0;
}

/* nearest_centroid (src/product_quantizer.cc:14-27): the first c whose l2sqr distance (the active
 * AVX2 kernel) is strictly below the best so far, starting from +inf; 0 when none is. */
size_t orc_nearest_centroid(const float* x, const float* centroids, size_t k, size_t dim) {
  size_t best = 0;
  float best_d = INFINITY;
  for (size_t c = 0; c < k; ++c) {
    const float d = orc_l2sqr_avx2(x, centroids + c * dim, dim);
    if (d < best_d) {
      best_d = d;
      best = c;
    }
  }
  return best;
}

/* centroid_table.h:94-144: dots accumulate x_j * c_j in order of j (unfused), then
 * d = ||c||^2 - 2*dot (or -dot for max inner product); the first strictly smaller d wins. A point
 * whose every d is NaN keeps index 0 (the caller's zero-initialized slot). */
static void nearest_t(const float* x, size_t n, const float* t, const float* norms, size_t k,
                      size_t dim, int max_ip, uint32_t* out, float* dots) {
  for (size_t p = 0; p < n; ++p) {
    const float* xp = x + p * dim;
    ct_dot_t(xp, t, k, dim, dots);
    float best = INFINITY;
    uint32_t arg = 0;
    for (size_t c = 0; c < k; ++c) {
      const float d = max_ip ? -dots[c] : norms[c] - 2.0f * dots[c];
      if (d < best) {
        best = d;
        arg = (uint32_t)c;
      }
    }
    out[p] = arg;
  }
}

void orc_nearest_batch(const float* x, size_t n, const float* cent, size_t k, size_t dim,
                       int max_inner_product, uint32_t* out, int nthreads) {
  float* t = transpose(cent, k, dim);
  float* norms = (float*)malloc(sizeof(float) * k);
  ct_norms(cent, k, dim, norms);
  const int nt = nthreads_or_max(nthreads);
#pragma omp parallel num_threads(nt)
  {
    float* dots = (float*)malloc(sizeof(float) * k);
#pragma omp for schedule(dynamic, 64)
    for (size_t p = 0; p < n; ++p) nearest_t(x + p * dim, 1, t, norms, k, dim, max_inner_product, out + p, dots);
    free(dots);
  }
  free(norms);
  free(t);
}

/* ------------------------------------------------------------------------------------------ */
/* Bounded top-k in lexicographic (distance, id) order                                        */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
  float d;
  uint64_t id;
} cand;

static int cand_less(cand a, cand b) { return a.d < b.d || (a.d == b.d && a.id < b.id); }

static void sift_up(cand* h, size_t i) {
  while (i > 0) {
    const size_t p = (i - 1) / 2;
    if (!cand_less(h[p], h[i])) break;
    const cand t = h[p];
    h[p] = h[i];
    h[i] = t;
    i = p;
  }
}

static void sift_down(cand* h, size_t n, size_t i) {
  for (;;) {
    size_t l = 2 * i + 1, big = i;
    if (l < n && cand_less(h[big], h[l])) big = l;
    if (l + 1 < n && cand_less(h[big], h[l + 1])) big = l + 1;
    if (big == i) return;
    const cand t = h[big];
    h[big] = h[i];
    h[i] = t;
    i = big;
  }
}

/* Max-heap of the `cap` lexicographically smallest candidates seen. */
static void topk_push(cand* h, size_t* size, size_t cap, cand c) {
  if (cap == 0) return;
  if (*size < cap) {
    h[(*size)++] = c;
    sift_up(h, *size - 1);
  } else if (cand_less(c, h[0])) {
    h[0] = c;
    sift_down(h, cap, 0);
  }
}

static int cand_cmp(const void* a, const void* b) {
  const cand x = *(const cand*)a, y = *(const cand*)b;
  return cand_less(x, y) ? -1 : (cand_less(y, x) ? 1 : 0);
}

static int bit_set(const uint64_t* bm, size_t i) { return (int)((bm[i >> 6] >> (i & 63)) & 1ULL); }

/* ------------------------------------------------------------------------------------------ */
/* FlatIndex                                                                                   */
/* ------------------------------------------------------------------------------------------ */

static float flat_dist(const float* q, const float* x, size_t dim, int l2) {
  float d = l2 ? orc_l2sqr_avx2(q, x, dim) : 1.0f - orc_dot_avx2(q, x, dim);
  return d == d ? d : INFINITY; /* src/flat_index.cc:88 */
}

int orc_flat_search(const float* base, size_t n, size_t dim, int metric, const float* queries,
                    size_t nq, size_t k, const uint64_t* row_bitmap, int nthreads,
                    uint32_t* out_rows, float* out_dist) {
  if (nq == 0 || k == 0) return 0;
  const int l2 = metric == ORC_L2;
  const int nt = nthreads_or_max(nthreads);
  const size_t cap = k < n ? k : n;
  enum { QB = 16 }; /* queries per pass over the rows (each query still sees rows in order) */
  const size_t nblocks = (nq + QB - 1) / QB;
#pragma omp parallel num_threads(nt)
  {
    cand* heaps = (cand*)malloc(sizeof(cand) * (cap + 1) * QB);
    size_t sizes[QB];
    float* qbuf = (float*)malloc(sizeof(float) * dim * QB);
#pragma omp for schedule(dynamic, 1)
    for (size_t blk = 0; blk < nblocks; ++blk) {
      const size_t q0 = blk * QB, nb = nq - q0 < QB ? nq - q0 : QB;
      for (size_t b = 0; b < nb; ++b) {
        memcpy(qbuf + b * dim, queries + (q0 + b) * dim, sizeof(float) * dim);
        if (metric == ORC_COSINE) normalize_one(qbuf + b * dim, dim); /* src/flat_index.cc:74-78 */
        sizes[b] = 0;
      }
      for (size_t i = 0; i < n; ++i) { /* src/flat_index.cc:84-96 */
        if (row_bitmap && !bit_set(row_bitmap, i)) continue;
        const float* x = base + i * dim;
        for (size_t b = 0; b < nb; ++b) {
          const cand c = {flat_dist(qbuf + b * dim, x, dim, l2), i};
          topk_push(heaps + b * (cap + 1), &sizes[b], cap, c);
        }
      }
      for (size_t b = 0; b < nb; ++b) {
        cand* heap = heaps + b * (cap + 1);
        const size_t qi = q0 + b;
        qsort(heap, sizes[b], sizeof(cand), cand_cmp); /* src/flat_index.cc:97 */
        for (size_t j = 0; j < k; ++j) {
          out_rows[qi * k + j] = j < sizes[b] ? (uint32_t)heap[j].id : UINT32_MAX;
          out_dist[qi * k + j] = j < sizes[b] ? heap[j].d : INFINITY;
        }
      }
    }
    free(qbuf);
    free(heaps);
  }
  return 0;
}

void orc_flat_pair_dist(const float* base, size_t dim, int metric, const float* queries,
                        size_t npairs, const uint64_t* qidx, const uint64_t* ridx, float* out) {
  float* qbuf = (float*)malloc(sizeof(float) * dim);
  for (size_t p = 0; p < npairs; ++p) {
    const float* q = queries + qidx[p] * dim;
    if (metric == ORC_COSINE) {
      memcpy(qbuf, q, sizeof(float) * dim);
      normalize_one(qbuf, dim);
      q = qbuf;
    }
    out[p] = flat_dist(q, base + ridx[p] * dim, dim, metric == ORC_L2);
  }
  free(qbuf);
}

/* ------------------------------------------------------------------------------------------ */
/* k-means and PQ training                                                                     */
/* ------------------------------------------------------------------------------------------ */

int orc_kmeans(const float* vectors, size_t n, size_t dim, size_t k, size_t iterations,
               size_t max_points_per_centroid, uint64_t seed, int nthreads, float* centroids) {
  if (k == 0 || dim == 0 || n < k) return -1; /* src/product_quantizer.cc:32-34 */
  orc_mt64 rng;
  orc_mt64_seed(&rng, seed);
  const float* x = vectors;
  float* sample = NULL;
  const size_t cap = k * (max_points_per_centroid > 1 ? max_points_per_centroid : 1);
  if (n > cap) { /* :42-54 */
    size_t* perm = (size_t*)malloc(sizeof(size_t) * n);
    for (size_t i = 0; i < n; ++i) perm[i] = i;
    for (size_t i = 0; i < cap; ++i) {
      const size_t j = i + (size_t)(orc_mt64_next(&rng) % (uint64_t)(n - i));
      const size_t t = perm[i];
      perm[i] = perm[j];
      perm[j] = t;
    }
    sample = (float*)malloc(sizeof(float) * cap * dim);
    for (size_t i = 0; i < cap; ++i) memcpy(sample + i * dim, vectors + perm[i] * dim, sizeof(float) * dim);
    free(perm);
    x = sample;
    n = cap;
  }
  { /* :57-65 */
    size_t* perm = (size_t*)malloc(sizeof(size_t) * n);
    for (size_t i = 0; i < n; ++i) perm[i] = i;
    for (size_t i = 0; i < k; ++i) {
      const size_t j = i + (size_t)(orc_mt64_next(&rng) % (uint64_t)(n - i));
      const size_t t = perm[i];
      perm[i] = perm[j];
      perm[j] = t;
      memcpy(centroids + i * dim, x + perm[i] * dim, sizeof(float) * dim);
    }
    free(perm);
  }
  uint32_t* assign = (uint32_t*)malloc(sizeof(uint32_t) * n);
  double* sums = (double*)malloc(sizeof(double) * k * dim);
  size_t* counts = (size_t*)malloc(sizeof(size_t) * k);
  for (size_t iter = 0; iter < iterations; ++iter) { /* :71-115 */
    orc_nearest_batch(x, n, centroids, k, dim, 0, assign, nthreads);
    memset(sums, 0, sizeof(double) * k * dim);
    memset(counts, 0, sizeof(size_t) * k);
    for (size_t i = 0; i < n; ++i) {
      const size_t c = assign[i];
      ++counts[c];
      for (size_t j = 0; j < dim; ++j) sums[c * dim + j] += (double)x[i * dim + j];
    }
    for (size_t c = 0; c < k; ++c) {
      if (counts[c] == 0) continue;
      for (size_t j = 0; j < dim; ++j)
        centroids[c * dim + j] = (float)(sums[c * dim + j] / (double)counts[c]);
    }
    for (size_t c = 0; c < k; ++c) { /* :95-114 empty-cluster split */
      if (counts[c] != 0) continue;
      size_t donor = 0;
      for (;;) {
        donor = (size_t)(orc_mt64_next(&rng) % (uint64_t)k);
        const double u = orc_mt64_canonical(&rng);
        if ((double)counts[donor] / (double)n * (double)k > u) break;
      }
      const float eps = 1.0f / 1024.0f;
      for (size_t j = 0; j < dim; ++j) {
        const float v = centroids[donor * dim + j];
        const float sign = (j % 2 == 0) ? 1.0f : -1.0f;
        centroids[c * dim + j] = v * (1.0f + sign * eps);
        centroids[donor * dim + j] = v * (1.0f - sign * eps);
      }
      counts[c] = counts[donor] / 2;
      counts[donor] -= counts[c];
    }
  }
  free(counts);
  free(sums);
  free(assign);
  free(sample);
  return 0;
}

int orc_pq_train(const float* x, size_t n, size_t dim, size_t m, size_t iterations, uint64_t seed,
                 int nthreads, float* codebook) {
  if (m == 0 || dim % m != 0 || n < 256) return -1; /* src/product_quantizer.cc:135-137 */
  const size_t dsub = dim / m;
  float* sub = (float*)malloc(sizeof(float) * n * dsub);
  for (size_t j = 0; j < m; ++j) {
    for (size_t i = 0; i < n; ++i) memcpy(sub + i * dsub, x + i * dim + j * dsub, sizeof(float) * dsub);
    const int rc = orc_kmeans(sub, n, dsub, 256, iterations, 256, seed + j, nthreads,
                              codebook + j * 256 * dsub);
    if (rc != 0) {
      free(sub);
      return rc;
    }
  }
  free(sub);
  return 0;
}

/* src/product_quantizer.cc:165-171: per sub-space the exact L2 table (centroid_table.h:65-75)
 * and its first minimum. */
static void pq_encode_one(const float* cbt, size_t m, size_t dsub, const float* x, uint8_t* code) {
  float dist[256];
  for (size_t j = 0; j < m; ++j) {
    ct_l2_t(x + j * dsub, cbt + j * 256 * dsub, 256, dsub, dist);
    code[j] = (uint8_t)orc_argmin_n(dist, 256);
  }
}

/* Codebook with every sub-space transposed: cbt[j][t][c]. */
static float* codebook_t(const float* codebook, size_t m, size_t dsub) {
  float* t = (float*)malloc(sizeof(float) * m * 256 * dsub);
  for (size_t j = 0; j < m; ++j)
    for (size_t c = 0; c < 256; ++c)
      for (size_t s = 0; s < dsub; ++s)
        t[j * 256 * dsub + s * 256 + c] = codebook[(j * 256 + c) * dsub + s];
  return t;
}

void orc_pq_encode(const float* codebook, size_t dim, size_t m, const float* x, size_t n,
                   uint8_t* codes, int nthreads) {
  const size_t dsub = dim / m;
  float* cbt = codebook_t(codebook, m, dsub);
  const int nt = nthreads_or_max(nthreads);
#pragma omp parallel for num_threads(nt) schedule(dynamic, 256)
  for (size_t i = 0; i < n; ++i) pq_encode_one(cbt, m, dsub, x + i * dim, codes + i * m);
  free(cbt);
}

void orc_pq_tables(const float* codebook, size_t dim, size_t m, const float* q, float* l2_table,
                   float* ip_table) {
  const size_t dsub = dim / m;
  float* cbt = codebook_t(codebook, m, dsub);
  for (size_t j = 0; j < m; ++j) {
    if (l2_table) ct_l2_t(q + j * dsub, cbt + j * 256 * dsub, 256, dsub, l2_table + j * 256);
    if (ip_table) ct_dot_t(q + j * dsub, cbt + j * 256 * dsub, 256, dsub, ip_table + j * 256);
  }
  free(cbt);
}

/* src/product_quantizer.cc:188-192 (adc_batch, :194-217, sums each code in the same order). */
static float adc_one(const float* table, size_t m, const uint8_t* code) {
  float sum = 0.0f;
  for (size_t j = 0; j < m; ++j) sum += table[j * 256 + code[j]];
  return sum;
}

void orc_pq_adc(const float* table, size_t m, const uint8_t* codes, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = adc_one(table, m, codes + i * m);
}

/* ------------------------------------------------------------------------------------------ */
/* IVF-PQ                                                                                      */
/* ------------------------------------------------------------------------------------------ */

void orc_ivfpq_precompute(const float* cents, const float* cb, size_t nlist, size_t dim, size_t m,
                          float* table) {
  const size_t dsub = dim / m; /* src/ivfpq_index.cc:117-127 */
  for (size_t l = 0; l < nlist; ++l) {
    for (size_t j = 0; j < m; ++j) {
      const float* cl = cents + l * dim + j * dsub;
      for (size_t c = 0; c < 256; ++c) {
        const float* r = cb + (j * 256 + c) * dsub;
        float v = 0.0f;
        for (size_t t = 0; t < dsub; ++t) v += r[t] * r[t] + 2.0f * cl[t] * r[t];
        table[(l * m + j) * 256 + c] = v;
      }
    }
  }
}

static int precompute_applies(int metric, size_t nlist, size_t m) {
  /* src/ivfpq_index.cc:74,114: L2 only, and only within 256 MiB. */
  return metric == ORC_L2 && nlist * m * 256 * sizeof(float) <= ((size_t)256 << 20);
}

int orc_ivfpq_train(const float* in, size_t n, size_t d, int metric, size_t nlist, size_t m,
                    size_t iterations, uint64_t seed, int nthreads, float* centroids,
                    float* codebook, float* precomputed) {
  if (n < nlist || n < 256 || m == 0 || d % m != 0) return -1; /* src/ivfpq_index.cc:145-146 */
  float* data = (float*)malloc(sizeof(float) * n * d);
  memcpy(data, in, sizeof(float) * n * d);
  if (metric == ORC_COSINE) orc_normalize(data, n, d); /* :154-156 */
  int rc = orc_kmeans(data, n, d, nlist, iterations, 256, seed, nthreads, centroids); /* :159-163 */
  if (rc != 0) {
    free(data);
    return rc;
  }
  if (metric == ORC_COSINE) orc_normalize(centroids, nlist, d); /* :164-167 */
  uint32_t* cell = (uint32_t*)malloc(sizeof(uint32_t) * n); /* :172-182 */
  orc_nearest_batch(data, n, centroids, nlist, d, metric == ORC_IP, cell, nthreads);
  float* res = data; /* residuals in place */
  for (size_t i = 0; i < n; ++i)
    for (size_t j = 0; j < d; ++j) res[i * d + j] = data[i * d + j] - centroids[cell[i] * d + j];
  free(cell);
  const size_t pq_n = n < 65536 ? n : 65536; /* :185-194 */
  if (pq_n < n) {
    orc_mt64 rng;
    orc_mt64_seed(&rng, seed + 2);
    float* tmp = (float*)malloc(sizeof(float) * d);
    for (size_t i = 0; i < pq_n; ++i) {
      const size_t j = i + (size_t)(orc_mt64_next(&rng) % (uint64_t)(n - i));
      memcpy(tmp, res + i * d, sizeof(float) * d);
      memcpy(res + i * d, res + j * d, sizeof(float) * d);
      memcpy(res + j * d, tmp, sizeof(float) * d);
    }
    free(tmp);
  }
  rc = orc_pq_train(res, pq_n, d, m, iterations, seed + 1, nthreads, codebook); /* :195-196 */
  free(data);
  if (rc != 0) return rc;
  if (precomputed && precompute_applies(metric, nlist, m)) { /* :197 */
    orc_ivfpq_precompute(centroids, codebook, nlist, d, m, precomputed);
    return 1;
  }
  return 0;
}

void orc_ivfpq_encode(const float* centroids, const float* codebook, size_t nlist, size_t d,
                      size_t m, int metric, const float* in, size_t n, int nthreads,
                      uint32_t* assign, uint8_t* codes, float* x_stored) {
  const float* x = in; /* src/ivfpq_index.cc:218-224 */
  float* normed = NULL;
  if (metric == ORC_COSINE) {
    normed = x_stored ? x_stored : (float*)malloc(sizeof(float) * n * d);
    memcpy(normed, in, sizeof(float) * n * d);
    orc_normalize(normed, n, d);
    x = normed;
  } else if (x_stored) {
    memcpy(x_stored, in, sizeof(float) * n * d);
  }
  orc_nearest_batch(x, n, centroids, nlist, d, metric == ORC_IP, assign, nthreads); /* :238 */
  const size_t dsub = d / m;
  float* cbt = codebook_t(codebook, m, dsub);
  const int nt = nthreads_or_max(nthreads);
#pragma omp parallel num_threads(nt)
  {
    float* residual = (float*)malloc(sizeof(float) * d);
#pragma omp for schedule(dynamic, 64)
    for (size_t i = 0; i < n; ++i) { /* :239-245 */
      const float* v = x + i * d;
      const float* c = centroids + (size_t)assign[i] * d;
      for (size_t j = 0; j < d; ++j) residual[j] = v[j] - c[j];
      pq_encode_one(cbt, m, dsub, residual, codes + i * m);
    }
    free(residual);
  }
  free(cbt);
  if (normed && normed != x_stored) free(normed);
}

static int ivf_ip(int metric) { return metric != ORC_L2; } /* src/ivfpq_index.cc:109 */

int orc_ivfpq_search(const orc_ivfpq* ix, const float* queries, size_t nq, size_t k,
                     size_t nprobe_req, size_t refine_factor, const uint64_t* pos_bitmap,
                     int nthreads, uint64_t* out_refs, float* out_dist) {
  const size_t d = ix->dim, nlist = ix->nlist, m = ix->m;
  for (size_t i = 0; i < nq * k; ++i) { /* src/ivfpq_index.cc:277-279 */
    out_refs[i] = UINT64_MAX;
    out_dist[i] = INFINITY;
  }
  if (k == 0) return 0;
  const size_t count = ix->offsets[nlist];
  size_t nprobe = nprobe_req < 1 ? 1 : nprobe_req; /* :286 */
  if (nprobe > nlist) nprobe = nlist;
  const int refine = refine_factor > 0 && ix->vectors != NULL; /* :303-308 */
  const size_t factor = refine ? refine_factor : 1;
  size_t keep = factor > count / (k > 1 ? k : 1) ? count : k * factor;
  if (keep > count) keep = count;
  if (keep == 0) return 0;
  const int ip = ivf_ip(ix->metric);
  const int use_pre = ix->precomputed != NULL && !ip;
  const size_t dsub = d / m;
  float* ct = transpose(ix->centroids, nlist, d);
  float* cbt = codebook_t(ix->codebook, m, dsub);
  const int nt = nthreads_or_max(nthreads);
#pragma omp parallel num_threads(nt)
  {
    float* buf = (float*)malloc(sizeof(float) * nlist);
    float* qbuf = (float*)malloc(sizeof(float) * d);
    float* residual = (float*)malloc(sizeof(float) * d);
    float* table = (float*)malloc(sizeof(float) * m * 256);
    float* qtable = (float*)malloc(sizeof(float) * m * 256);
    cand* probes = (cand*)malloc(sizeof(cand) * nlist);
    cand* heap = (cand*)malloc(sizeof(cand) * (keep + 1));
#pragma omp for schedule(dynamic, 1)
    for (size_t qi = 0; qi < nq; ++qi) {
      const float* q = queries + qi * d;
      if (ix->metric == ORC_COSINE) { /* :131-136 */
        memcpy(qbuf, q, sizeof(float) * d);
        normalize_one(qbuf, d);
        q = qbuf;
      }
      if (ip) { /* :289-300 */
        ct_dot_t(q, ct, nlist, d, buf);
        for (size_t l = 0; l < nlist; ++l) probes[l] = (cand){-buf[l], l};
      } else {
        ct_l2_t(q, ct, nlist, d, buf);
        for (size_t l = 0; l < nlist; ++l) probes[l] = (cand){buf[l], l};
      }
      qsort(probes, nlist, sizeof(cand), cand_cmp);
      if (ip) { /* :312-318 */
        for (size_t j = 0; j < m; ++j) ct_dot_t(q + j * dsub, cbt + j * 256 * dsub, 256, dsub, table + j * 256);
      } else if (use_pre) {
        for (size_t j = 0; j < m; ++j) ct_dot_t(q + j * dsub, cbt + j * 256 * dsub, 256, dsub, qtable + j * 256);
        for (size_t t = 0; t < m * 256; ++t) qtable[t] *= -2.0f;
      }
      size_t size = 0;
      for (size_t pi = 0; pi < nprobe; ++pi) { /* :326-360 */
        const size_t l = (size_t)probes[pi].id;
        const size_t b = ix->offsets[l], len = ix->offsets[l + 1] - b;
        if (len == 0) continue;
        float base = 0.0f;
        if (ip) {
          base = -probes[pi].d;
        } else if (use_pre) {
          base = probes[pi].d;
          const float* pre = ix->precomputed + l * m * 256;
          for (size_t t = 0; t < m * 256; ++t) table[t] = pre[t] + qtable[t];
        } else {
          const float* c = ix->centroids + l * d;
          for (size_t j = 0; j < d; ++j) residual[j] = q[j] - c[j];
          for (size_t j = 0; j < m; ++j) ct_l2_t(residual + j * dsub, cbt + j * 256 * dsub, 256, dsub, table + j * 256);
        }
        for (size_t i = 0; i < len; ++i) {
          const float s = adc_one(table, m, ix->codes + (b + i) * m);
          float dist = ip ? 1.0f - (base + s) : base + s;
          dist = dist == dist ? dist : INFINITY;
          if (pos_bitmap && !bit_set(pos_bitmap, b + i)) continue;
          topk_push(heap, &size, keep, (cand){dist, ((uint64_t)l << 32) | i});
        }
      }
      if (refine) { /* :363-373 */
        for (size_t j = 0; j < size; ++j) {
          const uint64_t ref = heap[j].id;
          const size_t pos = ix->offsets[ref >> 32] + (ref & 0xffffffffULL);
          const float* x = ix->vectors + pos * d;
          heap[j].d = ip ? 1.0f - orc_dot_avx2(q, x, d) : orc_l2sqr_avx2(q, x, d);
        }
      }
      qsort(heap, size, sizeof(cand), cand_cmp); /* :374-380 */
      const size_t nout = size < k ? size : k;
      for (size_t j = 0; j < nout; ++j) {
        out_refs[qi * k + j] = heap[j].id;
        out_dist[qi * k + j] = heap[j].d;
      }
    }
    free(heap);
    free(probes);
    free(qtable);
    free(table);
    free(residual);
    free(qbuf);
    free(buf);
  }
  free(cbt);
  free(ct);
  return 0;
}
