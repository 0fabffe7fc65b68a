/*
 * qvh — the C-ABI between Quiver's C++ indexes and the gfx950 (MI355X) kernels.
 *
 * This is the drop-in boundary: the host C++ classes (quiver::FlatIndex, quiver::IvfPqIndex,
 * quiver_amd/csrc/host/) keep the reference's public API and call these functions where the
 * reference runs its CPU scan loops. Only plain pointers and sizes cross it; no exceptions, no
 * C++ or torch types. Every function returns QVH_OK (0) or a negative status; the message of the
 * last failure on the calling thread is qvh_last_error().
 *
 * Conventions kept from the reference (include/quiver/common.h:25-29, flat_index.h:30-36):
 *   metric 0 = squared L2, 1 = inner product (distance 1 - <q,x>), 2 = cosine (1 - cos; rows and
 *   queries unit-normalized exactly as simd::normalize does, src/simd/dispatch.cc:119-135);
 *   results are ascending by distance; empty slots carry row/ref "all ones" and +infinity.
 * Ties between exactly equal distances are broken by the smaller row (or list ref); the reference
 * leaves that order to libstdc++ heap internals (src/internal/search_util.h:26-28).
 *
 * "Host" entry points take host buffers and return after the results are in host memory.
 * "_device" entry points take device pointers and enqueue on `stream` (NULL = the handle's own
 * stream) without synchronizing. Calls on one handle are serialized internally, and on the device
 * too: a call on another stream first waits for the handle's earlier work, and the handle's stream
 * then waits for it, so later calls (and qvh_*_sync) are ordered after it. Distinct handles may be
 * used from distinct threads concurrently. Buffers the library regrows or releases are freed
 * only after the device is idle.
 */
#ifndef QVH_H_
#define QVH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int qvh_status;
#define QVH_OK 0
#define QVH_EINVAL (-22)   /* bad argument (the reference throws quiver::Error for these) */
#define QVH_ENOMEM (-12)   /* device allocation failed */
#define QVH_EDEVICE (-5)   /* no usable HIP device, or a HIP runtime failure */
#define QVH_EUNSUPPORTED (-95)

#define QVH_METRIC_L2 0
#define QVH_METRIC_IP 1
#define QVH_METRIC_COSINE 2

#define QVH_EMPTY_ROW 0xFFFFFFFFu
#define QVH_EMPTY_REF 0xFFFFFFFFFFFFFFFFull

typedef struct qvh_flat qvh_flat;
typedef struct qvh_ivfpq qvh_ivfpq;

/* Message of the last failed call on this thread ("" if none). */
const char* qvh_last_error(void);

/* Diagnostic (no counterpart in the reference): the number of device allocations the library has
 * made in this process so far (every hipMalloc of its own buffers goes through one counter). Tests
 * use it to check that an entry point allocates nothing. */
qvh_status qvh_device_allocations(uint64_t* count);

/* Selects and initializes the HIP device used by handles created afterwards on this thread's
 * process (default: device 0, initialized on first use). Fails with QVH_EDEVICE when no gfx950
 * device is present. */
qvh_status qvh_init(int device);

/* The HIP device index that handles use (qvh_init's choice, else 0). No counterpart in the
 * reference: device-resident callers use it to check that their buffers live on that device. */
qvh_status qvh_get_device(int* device);

/* Writes the device name and the gfx target (e.g. "gfx950") into caller buffers. */
qvh_status qvh_device_info(char* name, size_t name_len, char* arch, size_t arch_len,
                           int* compute_units);

/* Unit-normalizes n rows of `dim` floats in place, bit-identical to the reference's
 * simd::normalize with the AVX2 kernels (src/simd/dispatch.cc:119-135,
 * src/simd/kernels_avx2.cc:58-83). Host buffers. */
qvh_status qvh_normalize(float* rows, uint64_t n, uint32_t dim);

/* ------------------------------------------------------------------------------------------ *
 * Flat exact search: replaces the per-query scan of FlatIndex::search_one
 * (src/flat_index.cc:69-107) under FlatIndex::search_batch (src/flat_index.cc:126-140).
 * ------------------------------------------------------------------------------------------ */

/* FlatIndex(dim, metric) (src/flat_index.cc:41-47): an empty device-resident row store. */
qvh_status qvh_flat_create(uint32_t dim, int metric, qvh_flat** out);
void qvh_flat_destroy(qvh_flat* flat);

/* The append step of FlatIndex::add (src/flat_index.cc:62-65): copies n rows to the device
 * (normalizing them for cosine). `stored_out` (nullable, n*dim floats) receives the rows as
 * stored, i.e. normalized for cosine, for the host copy the C++ class keeps. */
qvh_status qvh_flat_append(qvh_flat* flat, const float* rows, uint64_t n, float* stored_out);

/* Appends n rows that are already in stored form (cosine rows unit-normalized), as
 * FlatIndex::load installs the VECT section (src/flat_index.cc:155-176). */
qvh_status qvh_flat_append_stored(qvh_flat* flat, const float* rows, uint64_t n);

/* Number of stored rows. */
uint64_t qvh_flat_size(const qvh_flat* flat);

/* The scan of FlatIndex::search_batch (src/flat_index.cc:84-106) for nq raw queries (normalized
 * here for cosine, as search_one does at :74-78). `row_bitmap` (nullable, ceil(size/64) words,
 * bit r of word r/64 set = row r admitted) is the Filter materialized over rows (:85): unless it
 * admits every row (then it is no filter), the scan runs over the list of admitted rows only, while
 * their contiguous copy stays within 4 GiB (else it tests the bitmap over every row).
 * Outputs: nq*k rows (QVH_EMPTY_ROW when fewer than k rows are admitted) and distances (+inf). */
qvh_status qvh_flat_search(qvh_flat* flat, const float* queries, uint64_t nq, uint32_t k,
                           const uint64_t* row_bitmap, uint32_t* out_rows, float* out_dist);

/* Exact top-k over the listed rows only: HnswIndex::search_exact's scan over the labels a
 * selective filter admits (src/hnsw_index.cc:722-739, taken when the filter's cardinality is at
 * most exact_scan_threshold x live nodes, src/hnsw_index.cc:755-760), on a device row store whose
 * rows are the graph's node ids. `rows` (host, any order; repeats count once) must all be below
 * the stored row count (else QVH_EINVAL). Outputs as qvh_flat_search. */
qvh_status qvh_flat_search_rows(qvh_flat* flat, const float* queries, uint64_t nq, uint32_t k,
                                const uint32_t* rows, uint64_t nrows, uint32_t* out_rows,
                                float* out_dist);

/* Same, on device-resident buffers, enqueued on `stream` (a hipStream_t; NULL = the handle's).
 * The device bitmap is tested per tile over every row. */
qvh_status qvh_flat_search_device(qvh_flat* flat, const float* d_queries, uint64_t nq,
                                  uint32_t k, const uint64_t* d_row_bitmap, uint32_t* d_out_rows,
                                  float* d_out_dist, void* stream);

/* qvh_flat_search_device with the admitted rows given as a device list instead of a bitmap: no
 * counterpart in the reference (its search takes the Filter on the host, src/flat_index.cc:85);
 * for device-resident callers, whose filter the host turns into rows once. `d_row_list` holds
 * `nrows` rows in ascending order, without repeats, each below the stored row count (at most that
 * count, else QVH_EINVAL; rows past the last stored one are read as the last). The scan reads only
 * the listed rows, as qvh_flat_search does with a host filter; all stored rows listed is no filter.
 * Where the listed-row scan does not apply (its copy above 4 GiB, or a k it does not serve) the list
 * becomes a device bitmap first. Enqueued on `stream` (NULL = the handle's). */
qvh_status qvh_flat_search_device_rows(qvh_flat* flat, const float* d_queries, uint64_t nq,
                                       uint32_t k, const uint32_t* d_row_list, uint64_t nrows,
                                       uint32_t* d_out_rows, float* d_out_dist, void* stream);

/* qvh_flat_search_device without any allocation: no counterpart in the reference; for callers that
 * cannot allocate device memory during a search (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, kernels and results as qvh_flat_search_device;
 * the workspace (prepared queries, norms, bounds, partial lists, counters) comes from a fixed
 * 64 MiB array in device memory that each GPU the library runs on holds until the process ends. A
 * search that needs more (many queries, or few queries with a large k) fails with QVH_EINVAL
 * before anything is enqueued. All calls on one GPU share that GPU's array; the library orders them
 * on the device (each call's stream waits for the previous call's last launch, through an event),
 * so calls on different handles or streams take the array in turn. Under HIP graph capture that
 * ordering is left to the caller. Each call clears what must start at zero itself. */
qvh_status qvh_flat_search_device_noalloc(qvh_flat* flat, const float* d_queries, uint64_t nq,
                                          uint32_t k, const uint64_t* d_row_bitmap,
                                          uint32_t* d_out_rows, float* d_out_dist, void* stream);

/* Waits for all work enqueued on the handle (its stream, which every call joins). */
qvh_status qvh_flat_sync(qvh_flat* flat);

/* Measurement hook (no counterpart in the reference): when enabled, each search records HIP
 * events around its three stages (query prep, fused scan, merge + exact re-score) on the stream
 * the kernels run on; qvh_flat_last_timing waits for the last search and returns the stage
 * durations in milliseconds and the number of row splits the scan used. */
qvh_status qvh_flat_set_timing(qvh_flat* flat, int enable);
qvh_status qvh_flat_last_timing(qvh_flat* flat, float* prep_ms, float* scan_ms, float* merge_ms,
                                uint32_t* nsplit);

/* Diagnostic (no counterpart in the reference): the number of queries of the last search on the
 * MFMA scan that the merge handed to the exact kernel, because the re-scored selection could not be
 * certified (the k-th exact distance was not below the last selected GEMM-form distance minus the
 * query's rounding bound) or, for k above the shared-bound lists, a split's 32-entry list ran out
 * before the selection ended; 0 for searches on the other kernels. Waits for the last search. */
qvh_status qvh_flat_last_fallbacks(qvh_flat* flat, uint32_t* count);

/* ------------------------------------------------------------------------------------------ *
 * IVF-PQ: replaces the encode step of IvfPqIndex::Impl::add (src/ivfpq_index.cc:208-271) and
 * the query path of IvfPqIndex::Impl::search_into (src/ivfpq_index.cc:275-381). Lists live on
 * the device in CSR order (the LOFF/CODE/VECT layout of src/ivfpq_index.cc:479-503); labels stay
 * with the caller, who maps refs back to them.
 * ------------------------------------------------------------------------------------------ */

/* IvfPqIndex(params) (src/ivfpq_index.cc:95-103): dim, metric, nlist, m (dim % m == 0),
 * store_vectors. */
qvh_status qvh_ivfpq_create(uint32_t dim, int metric, uint32_t nlist, uint32_t m, int store_vectors,
                            qvh_ivfpq** out);
void qvh_ivfpq_destroy(qvh_ivfpq* ivf);

/* Installs the trained state, as Impl::train commits it (src/ivfpq_index.cc:199-205): coarse
 * centroids [nlist][dim] and PQ codebook [m][256][dim/m]. With use_precomputed (L2 only) the
 * device builds the nlist x m x 256 term table of Impl::precompute (src/ivfpq_index.cc:112-129). */
qvh_status qvh_ivfpq_set_trained(qvh_ivfpq* ivf, const float* centroids, const float* codebook,
                                 int use_precomputed);
/* Copies the precomputed table [nlist][m][256] to the host. */
qvh_status qvh_ivfpq_precomputed(qvh_ivfpq* ivf, float* out);

/* The encode step of Impl::add (src/ivfpq_index.cc:218-247): cells and PQ codes of n vectors,
 * without storing them: assign[n] (nullable), codes[n][m] (nullable), stored_out[n][dim] = the
 * vectors as stored (normalized for cosine; nullable). It runs on a workspace and stream of its own
 * and does not take the handle's lock, so searches on the same handle proceed meanwhile, as they do
 * during the reference's encode (which holds no index lock). Concurrent encodes on one handle are
 * serialized with each other. */
qvh_status qvh_ivfpq_encode(qvh_ivfpq* ivf, const float* x, uint64_t n, uint32_t* assign,
                            uint8_t* codes, float* stored_out);

/* The append step of Impl::add (src/ivfpq_index.cc:249-270, the part the reference runs under
 * the exclusive lock): stores n entries that qvh_ivfpq_encode produced, each after its list's
 * existing entries in batch order. assign[n] and codes[n][m] are required; vectors[n][dim] (the
 * stored form, normalized for cosine) is required when the index stores vectors and ignored
 * otherwise. A cell out of range or a list that would pass 2^32 entries is rejected (QVH_EINVAL)
 * before anything changes. */
qvh_status qvh_ivfpq_append(qvh_ivfpq* ivf, const uint32_t* assign, const uint8_t* codes,
                            const float* vectors, uint64_t n);

/* Impl::add (src/ivfpq_index.cc:208-271) in one call: encodes n vectors and appends them to their
 * lists in input order, holding the handle's lock throughout. assign_out[n] (nullable) receives
 * each vector's list, which the caller needs to place its labels. */
qvh_status qvh_ivfpq_add(qvh_ivfpq* ivf, const float* x, uint64_t n, uint32_t* assign_out);

/* Installs whole lists into an empty trained index, as IvfPqIndex::load does from the LOFF /
 * CODE / VECT sections (src/ivfpq_index.cc:547-573): offsets [nlist + 1], codes [count][m] and,
 * with store_vectors, vectors [count][dim], all in list order. */
qvh_status qvh_ivfpq_set_lists(qvh_ivfpq* ivf, const uint64_t* offsets, const uint8_t* codes,
                               const float* vectors);

uint64_t qvh_ivfpq_size(const qvh_ivfpq* ivf);
/* CSR offsets [nlist + 1] of the lists. */
qvh_status qvh_ivfpq_list_offsets(qvh_ivfpq* ivf, uint64_t* offsets);
/* Stored codes [count][m] and vectors [count][dim] (nullable each) in CSR order. */
qvh_status qvh_ivfpq_lists(qvh_ivfpq* ivf, uint8_t* codes, float* vectors);

/* search_into for nq raw queries (normalized here for cosine): nprobe clamped to [1, nlist],
 * keep = min(size, k * refine_factor) with refine only when vectors are stored,
 * `pos_bitmap` (nullable, ceil(size/64) words over CSR positions) is the Filter. Outputs nq*k
 * refs ((list << 32) | offset in list, QVH_EMPTY_REF when empty) and distances. */
qvh_status qvh_ivfpq_search(qvh_ivfpq* ivf, const float* queries, uint64_t nq, uint32_t k,
                            uint32_t nprobe, uint64_t refine_factor, const uint64_t* pos_bitmap,
                            uint64_t* out_refs, float* out_dist);
/* Same on device-resident buffers, enqueued on `stream` (NULL = the handle's). */
qvh_status qvh_ivfpq_search_device(qvh_ivfpq* ivf, const float* d_queries, uint64_t nq,
                                   uint32_t k, uint32_t nprobe, uint64_t refine_factor,
                                   const uint64_t* d_pos_bitmap, uint64_t* d_out_refs,
                                   float* d_out_dist, void* stream);
qvh_status qvh_ivfpq_sync(qvh_ivfpq* ivf);
/* Diagnostic (no counterpart in the reference): the number of queries of the last search (L2 with
 * the precomputed table, which ranks by an approximate sum and re-scores the best) whose ranking
 * could not be certified against the rounding bound and was recomputed with the reference's sums
 * for every probed code; 0 for other searches. Waits for the last search. */
qvh_status qvh_ivfpq_last_fallbacks(qvh_ivfpq* ivf, uint32_t* count);
/* Measurement hook (no counterpart in the reference). Level 1: HIP events around the probe
 * selection (query prep, coarse scores, top-nprobe, the ranking certificate's bounds) and the list
 * scan of each search (the scan kernel, which also re-ranks with refine; not the rescan of
 * uncertified queries that follows). Level 2
 * adds, after the scan, a count of the PQ code bytes the scan had to read (sum over queries and
 * probed lists of len * m), which qvh_ivfpq_last_timing returns in code_bytes (nullable). */
qvh_status qvh_ivfpq_set_timing(qvh_ivfpq* ivf, int enable);
qvh_status qvh_ivfpq_last_timing(qvh_ivfpq* ivf, float* select_ms, float* scan_ms,
                                 uint64_t* code_bytes);

/* ------------------------------------------------------------------------------------------ *
 * Nearest-centroid assignment for k-means (src/product_quantizer.cc:72-77), restating
 * CentroidTable::nearest_batch (src/internal/centroid_table.h:94-144) bit for bit: a device
 * resident point set assigned repeatedly against changing centroids.
 * ------------------------------------------------------------------------------------------ */
typedef struct qvh_points qvh_points;
qvh_status qvh_points_create(const float* x, uint64_t n, uint32_t dim, qvh_points** out);
void qvh_points_destroy(qvh_points* points);
qvh_status qvh_points_nearest(qvh_points* points, const float* centroids, uint32_t k,
                              int max_inner_product, uint32_t* out_assign);

/* ------------------------------------------------------------------------------------------ *
 * ProductQuantizer (include/quiver/quantizer.h:59-114, src/product_quantizer.cc:119-217) and
 * nearest_centroid (src/product_quantizer.cc:14-27), over batches: the reference's per-vector
 * methods are the n = 1 case. Every sum follows the reference's float order, so codes, tables,
 * ADC sums and indices are bit-identical. Host buffers; each call returns when its outputs are
 * written.
 * ------------------------------------------------------------------------------------------ */
typedef struct qvh_pq qvh_pq;

/* ProductQuantizer(dim, m) + set_centroids (src/product_quantizer.cc:119-124,155-163): the
 * codebook [m][256][dim/m] goes to the device. dim % m must be 0. */
qvh_status qvh_pq_create(uint32_t dim, uint32_t m, const float* codebook, qvh_pq** out);
void qvh_pq_destroy(qvh_pq* pq);

/* ProductQuantizer::encode of n vectors [n][dim] (src/product_quantizer.cc:165-171): codes [n][m],
 * per sub-space the first of the 256 codewords with the smallest in-order sum of squared
 * differences (CentroidTable::l2 + argmin, src/internal/centroid_table.h:65-75,155-170). */
qvh_status qvh_pq_encode(qvh_pq* pq, const float* x, uint64_t n, uint8_t* codes);

/* ProductQuantizer::decode of n codes [n][m] into [n][dim] (src/product_quantizer.cc:173-178). */
qvh_status qvh_pq_decode(qvh_pq* pq, const uint8_t* codes, uint64_t n, float* out);

/* compute_l2_table (inner_product = 0) or compute_ip_table (1) of nq queries [nq][dim]
 * (src/product_quantizer.cc:180-186): tables [nq][m][256]. */
qvh_status qvh_pq_tables(qvh_pq* pq, const float* queries, uint64_t nq, int inner_product,
                         float* tables);

/* ProductQuantizer::adc_batch (src/product_quantizer.cc:194-217; adc is n = 1): out[i] = the sum
 * over j of table[j * 256 + codes[i][j]], in order of j, for one table [m][256]. */
qvh_status qvh_pq_adc(qvh_pq* pq, const float* table, const uint8_t* codes, uint64_t n, float* out);

/* nearest_centroid (src/product_quantizer.cc:14-27) of n points [n][dim] against k centroids
 * [k][dim]: the first index with the smallest simd::l2sqr distance (AVX2 order), 0 when no
 * distance is below +infinity. */
qvh_status qvh_nearest_centroid(const float* x, uint64_t n, const float* centroids, uint32_t k,
                                uint32_t dim, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* QVH_H_ */
