// Flat exact search on gfx950: the FlatIndex::search_batch scan (src/flat_index.cc:69-140).
//
// Pipeline for one call:
//   1. prep:  queries -> device, unit-normalized for cosine (exact simd::normalize order),
//             zero-padded to DP floats, ||q||^2.
//   2. scan:  fp32 MFMA GEMM (v_mfma_f32_32x32x2_f32) of a 32-query column block held in VGPRs
//             against 64-row base tiles staged through LDS (double buffered, padded stride),
//             with the distance epilogue ||q||^2 + ||x||^2 - 2<q,x> (or 1 - <q,x>) and a per-lane
//             register top-KL list fused in, so the nq x n distance matrix never reaches HBM.
//             Each (query block, row split) is one workgroup; each query ends with 2 * nsplit
//             sorted lists of KL candidates.
//   3. merge: one wave per query pops the KL best candidates of those lists, re-scores them with
//             the reference's exact AVX2-order arithmetic, and writes the k best by
//             (exact distance, row).
// The GEMM form differs from the reference's sum of squared differences only in rounding; the
// re-score makes every returned distance bit-identical to the reference's for that row, and KL > k
// keeps a margin of near-tied candidates for the re-score to choose from.
#include <algorithm>
#include <cstring>
#include <vector>
#include <type_traits>

#include <rocprim/device/device_segmented_radix_sort.hpp>

#include "common.hpp"
#include "exact.hpp"
#include "select.hpp"

namespace qvh {
void launch_normalize_rows(float* d_rows, uint64_t n, uint32_t dim, hipStream_t stream);
}

namespace {

using namespace qvh;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 8;                                 // 2 waves per SIMD
constexpr int kThreads = kWaves * 64;
constexpr int kTileRows = 64;                             // two 32-row MFMA blocks
constexpr int kQueriesPerBlock = kWaves * 32;             // each wave owns 32 queries
constexpr int kMaxListsPerLane = 8;                       // merge: lists per lane
constexpr uint32_t kMaxSplits = 64 * kMaxListsPerLane / 2;
constexpr int kMaxDp = 128;                               // register-resident query width

struct ScanArgs {
  const float* X;           // [cap][DP] rows as stored, zero padded
  const float* xnorm;       // [cap] ||x||^2
  uint64_t n;
  const float* Q;           // [nq][DP] prepared queries
  const float* qnorm;       // [nq] ||q||^2
  uint32_t nq;
  const uint64_t* bitmap;   // admitted rows, or null
  int l2;
  uint32_t nsplit;
  uint32_t qblocks;
  uint64_t rows_per_split;  // multiple of kTileRows (of 32 for the ring scan)
  float* part_d;            // [nq][2*nsplit][KL]
  uint32_t* part_r;
  uint32_t* qthr;           // shared prune bounds (ordered float bits, +inf at the start): the
                            // register and chunked scans kScanBoundStride words per query, the
                            // ring scan kRingBoundStride
  int share;                // 0: every lane list keeps its own KL best (k > KL: no shared bound)
  uint32_t dp;              // row width (the chunked scan; the register scan has it as DP)
  int rowsplit;             // register scan, unfiltered, at most 128 queries: two waves per query group
  int bound_slots;          // register scan: publish and read the per-query bound slots
  // Register scan with 32-entry lists for k above 21 (the wide merge takes R = k + max(16, k / 2)
  // keys): when nonzero, c = ceil(R / 2) <= 32, and the shared bound is the larger of the lane
  // pair's c-th entries (2c >= R rows of the pair lie at or below it, so it bounds the R-th best).
  uint32_t share_rank;
  // Launch gate: when set, the launch does nothing unless (*gate != 0) == (gate_want != 0), read
  // once at the start. Two list lengths are launched back to back and the device picks one.
  const uint32_t* gate;
  uint32_t gate_want;
};

__device__ __forceinline__ bool gate_closed(const uint32_t* gate, uint32_t want) {
  return gate != nullptr && ((*gate != 0u) != (want != 0u));
}

constexpr int kShareEvery = 8;  // chunked scan: tiles between exchanges of the shared per-query bound
// The MFMA scan's words per query in ScanArgs::qthr: word 0 the union bound, words kScanSlotBase
// and up the bound slots (one per list source, at most 32), on the query's second 128-byte line.
constexpr uint32_t kScanBoundStride = 64;
constexpr uint32_t kScanSlotBase = 32;
constexpr int kScanSlots = 32;
// Splits per query up to which the row-split form of the register scan (four lists per split and
// query) uses the bound slots: with more, the atomics of its many lists on the query's slot line
// queue up (1M x 128, 128 queries on 256 splits: 0.39 ms without the slots, 0.49 ms with them). The
// register scan's full-block form (two lists per split and query) uses them at any split count
// (10,000 queries on 32 splits: 21.50 ms without, 21.23 ms with; 512 queries on 256 splits 1.33 ->
// 1.23 ms, 1,024 on 256 2.46 -> 2.30 ms, 2,048 on 128 4.71 -> 4.26 ms).
constexpr uint64_t kScanSlotMaxSplits = 64;

/// Tiles after which the register scan exchanges bounds: 0, 1, 3, 7, 15, 31 and 63 (the lists' first
/// rows move a bound the most, and a split of a few tiles would otherwise never take the shared
/// one), then every 64. An exchange stalls the wave for a device-scope round trip, and late in a
/// split the bounds move little (1M x 128, 10,000 queries: every 8 tiles 21.07 ms, every 16 20.58,
/// every 32 20.30, this schedule 20.22, every 128 after 127 20.21).
__device__ __forceinline__ bool scan_share_after(uint32_t t) {
  return t < 64 ? (t & (t + 1)) == 0 : t % 64 == 63;
}
constexpr int kQueueCap = 20;   // queued candidates per lane before a wave-wide flush

/// Inserts (d, r) into the ascending list (Ld, Lr) in (distance, row) order, dropping the last.
template <int KL>
__device__ __forceinline__ void list_insert(float (&Ld)[KL], uint32_t (&Lr)[KL], float d, uint32_t r) {
#pragma unroll
  for (int x = 0; x < KL; ++x) {
    const bool lt = (d < Ld[x]) | ((d == Ld[x]) & (r < Lr[x]));
    const float td = Ld[x];
    const uint32_t tr = Lr[x];
    Ld[x] = lt ? d : td;
    Lr[x] = lt ? r : tr;
    d = lt ? td : d;
    r = lt ? tr : r;
  }
}

/// Inserts (d, r) into the sorted list (the caller has checked d <= Ld[KL - 1]) for a lane whose
/// candidates come in increasing row order: a listed entry of equal distance then holds a smaller
/// row and stays ahead, so the new entry goes before the first entry of larger distance or the
/// first empty one (an empty entry, +inf and QVH_EMPTY_ROW, gives way to a row at +inf). Every
/// compare reads the old list and every entry's new value depends on its own compare and its
/// neighbour's, so the insertion is one parallel step rather than a chain through the list.
template <int KL>
__device__ __forceinline__ void list_insert_ordered(float (&Ld)[KL], uint32_t (&Lr)[KL], float d, uint32_t r) {
  bool lt[KL];
#pragma unroll
  for (int x = 0; x < KL; ++x) lt[x] = (d < Ld[x]) | (Lr[x] == QVH_EMPTY_ROW);
#pragma unroll
  for (int x = KL - 1; x > 0; --x) {
    Ld[x] = lt[x] ? (lt[x - 1] ? Ld[x - 1] : d) : Ld[x];
    Lr[x] = lt[x] ? (lt[x - 1] ? Lr[x - 1] : r) : Lr[x];
  }
  Ld[0] = lt[0] ? d : Ld[0];
  Lr[0] = lt[0] ? r : Lr[0];
}

/// Sorts 16 values ascending in registers (a bitonic network of 80 compare-exchanges).
__device__ __forceinline__ void sort16_u32(uint32_t (&v)[16]) {
#pragma unroll
  for (int size = 2; size <= 16; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int l = i ^ stride;
        if (l > i) {
          const uint32_t lo = min(v[i], v[l]), hi = max(v[i], v[l]);
          const bool up = (i & size) == 0;
          v[i] = up ? lo : hi;
          v[l] = up ? hi : lo;
        }
      }
    }
  }
}

/// The K-th smallest of the 32 values held 16 by this lane and 16 by its partner (lane ^ 32),
/// the same in both lanes. K = 32 is the maximum; below it both halves are sorted and the K-th
/// smallest of the union is min over i of max(S[i - 1], P[K - 1 - i]) (i values from this lane's
/// sorted S, the rest from the partner's P).
template <int K>
__device__ __forceinline__ uint32_t pair_kth_smallest(uint32_t (&v)[16]) {
  static_assert(K >= 1 && (K <= 16 || K == 32), "K-th of 32");
  if constexpr (K == 32) {
    uint32_t m = v[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) m = max(m, v[i]);
    return max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 32, 64)));
  } else {
    sort16_u32(v);
    uint32_t p[K];
#pragma unroll
    for (int i = 0; i < K; ++i) p[i] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v[i]), 32, 64));
    uint32_t r = min(v[K - 1], p[K - 1]);
#pragma unroll
    for (int i = 1; i < K; ++i) r = min(r, max(v[i - 1], p[K - 1 - i]));
    return r;
  }
}

/// Appends a lane's passing candidates of one 32x32 distance block to its queue (entry e at
/// s_qd / s_qr[e * kThreads + tid], room for 16 left by the caller). Register r holds row
/// row0 + 8*(r/4) + r%4; it passes when lane_ok, !(d > thr) (ties and NaN pass) and, with MASKED,
/// bit 8*(r/4) + r%4 of lane_bits is set. An element that no lane of the wave passes costs a
/// compare and a skipped branch.
template <bool MASKED>
__device__ __forceinline__ void queue_block(const f32x16& acc, float thr, bool lane_ok, uint32_t lane_bits,
                                            uint32_t row0, int tid, int& qcount, float* s_qd, uint32_t* s_qr) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int bit = 8 * (r >> 2) + (r & 3);
    bool p = lane_ok && !(acc[r] > thr);
    if (MASKED) p = p && ((lane_bits >> bit) & 1u);
    if (__builtin_amdgcn_ballot_w64(p)) {
      if (p) {
        s_qd[qcount * kThreads + tid] = acc[r];
        s_qr[qcount * kThreads + tid] = row0 + static_cast<uint32_t>(bit);
        ++qcount;
      }
    }
  }
}

/// A scan lane's selection state: its list of the KL best (distance, row) among the rows it has
/// seen, its candidate queue (CAP entries in LDS, entry-major: entry e of thread t at e * kThreads
/// + t, so lanes appending at different depths never share a bank) and its prune threshold.
/// Candidates are appended in row order and inserted into the list by a wave-wide flush. Shared
/// by the scan kernels.
template <int KL, int CAP>
struct LaneScan {
  float Ld[KL];
  uint32_t Lr[KL];
  int qcount;
  // Prune threshold: the smaller of this lane's KL-th best and the shared per-query value. Any
  // list's KL-th best bounds the KL-th best of the union of all lists, so candidates above it can
  // never be among the query's KL best (equal distances pass: ties are decided by row).
  float pthr;
  int tid;

  __device__ __forceinline__ void init(int thread, float thr0) {
#pragma unroll
    for (int x = 0; x < KL; ++x) {
      Ld[x] = __builtin_huge_valf();
      Lr[x] = QVH_EMPTY_ROW;
    }
    qcount = 0;
    pthr = thr0;
    tid = thread;
  }

  /// All lanes of the wave together: queued candidates into the lists (NaN becomes +inf). s_qd and
  /// s_qr are the work-group's queue arrays (CAP * kThreads entries).
  __device__ __forceinline__ void flush(const float* s_qd, const uint32_t* s_qr) {
    int m = qcount;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
    for (int e = 0; e < m; ++e) {
      if (e < qcount) {
        float v = s_qd[e * kThreads + tid];
        v = v == v ? v : __builtin_huge_valf();
        if (v <= Ld[KL - 1]) list_insert_ordered<KL>(Ld, Lr, v, s_qr[e * kThreads + tid]);
      }
    }
    qcount = 0;
  }

  /// Exchange through the per-query value *qthr (null for lanes past the last query). The two
  /// lanes of a query (j, j + 32) hold disjoint rows: their union has KL candidates at or below
  /// max(own[KL/2-1], other[KL/2-1]) as well as below either list's KL-th.
  __device__ __forceinline__ void share(uint32_t* qthr, int h, int j) {
    const float own_k = Ld[KL - 1], own_h = Ld[KL / 2 - 1];
    const float oth_k = __shfl_xor(own_k, 32, 64), oth_h = __shfl_xor(own_h, 32, 64);
    float t = fminf(fminf(own_k, oth_k), fmaxf(own_h, oth_h));
    if (qthr) {
      uint32_t g = 0;
      if (h == 0) g = atomicMin(qthr, float_to_ordered(t));
      g = __shfl(g, j, 64);
      t = fminf(t, ordered_to_float(g));
    }
    pthr = fminf(pthr, t);
  }

  /// One 32x32 block of distances (register r: row 8*(r/4) + 4*h + r%4 of the block, rows
  /// row0 + 8*(r/4) + r%4 with row0 = block's first row + 4*h); lane_bits: admission of those rows
  /// (bit 8*(r/4) + r%4), tested when `masked` (wave-uniform). Per lane the rows visited increase,
  /// so ties resolve to the smaller row.
  __device__ __forceinline__ void block(const f32x16& acc, uint32_t lane_bits, bool masked, bool qvalid,
                                        uint32_t row0, float* s_qd, uint32_t* s_qr) {
    // Pass test: !(d > thr). Ties pass (a tied row may still win on row number), and so does
    // NaN, which the flush turns into +inf as the reference does.
    const float thr = fminf(pthr, Ld[KL - 1]);
    bool any = false;
    if (!masked) {
      // One test of the smallest distance (fminf skips NaN; all-NaN gives NaN, which passes).
      float m = acc[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) m = fminf(m, acc[r]);
      any = !(m > thr);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        any = any || (!(acc[r] > thr) && ((lane_bits >> (8 * (r >> 2) + (r & 3))) & 1u));
      }
    }
    // Lanes past the last query never queue: their zero query makes every inner-product
    // distance 1 exactly, a tie with their own list that would admit every row.
    any = any && qvalid;
    if (__builtin_amdgcn_ballot_w64(any)) {
      if (__builtin_amdgcn_ballot_w64(qcount > CAP - 16)) flush(s_qd, s_qr);
      if (masked) {
        queue_block<true>(acc, thr, any, lane_bits, row0, tid, qcount, s_qd, s_qr);
      } else {
        queue_block<false>(acc, thr, any, lane_bits, row0, tid, qcount, s_qd, s_qr);
      }
    }
  }

  /// The two blocks of a 64-row tile starting at tile_row0, `left` of its rows inside the split,
  /// `admit` the filter's bits for the tile (all ones without a filter).
  __device__ __forceinline__ void tile(const f32x16& acc0, const f32x16& acc1, uint64_t tile_row0, uint64_t left,
                                       uint64_t admit, bool filter, bool qvalid, int h, float* s_qd, uint32_t* s_qr) {
    if (left < 64) admit &= (1ull << left) - 1;
    const bool masked = filter || left < 64;
    block(acc0, static_cast<uint32_t>(admit) >> (4 * h), masked, qvalid, static_cast<uint32_t>(tile_row0 + 4 * h),
          s_qd, s_qr);
    block(acc1, static_cast<uint32_t>(admit >> 32) >> (4 * h), masked, qvalid,
          static_cast<uint32_t>(tile_row0 + 32 + 4 * h), s_qd, s_qr);
  }

  /// The lane's list into part_d / part_r at offset o.
  __device__ __forceinline__ void store(float* part_d, uint32_t* part_r, size_t o) const {
#pragma unroll
    for (int x = 0; x < KL; ++x) {
      part_d[o + x] = Ld[x];
      part_r[o + x] = Lr[x];
    }
  }
};

/// Row split and query block of work-group blockIdx.x. Work-group w runs on XCD w % 8; each XCD
/// gets its own row splits, so the work-groups resident on one XCD at a time stream the same base
/// rows through that XCD's L2.
__device__ __forceinline__ void scan_block_coords(const ScanArgs& a, uint32_t& qb, uint32_t& split) {
  const uint32_t wg = blockIdx.x;
  if (a.nsplit % 8 == 0) {
    const uint32_t x = wg % 8, li = wg / 8;
    split = (li / a.qblocks) * 8 + x;
    qb = li % a.qblocks;
  } else {
    split = wg / a.qblocks;
    qb = wg % a.qblocks;
  }
}

// MODE: 0 every row of a.X (the store, or a contiguous copy of listed rows: candidates then carry
// positions in the list, which the merge maps to rows), 1 rows admitted by a bitmap (tested per tile).
// RS (row split, small batches): the block serves 128 queries, and the two waves of a 32-query group
// take the two 32-row halves of every tile, so a batch of 32 queries keeps two SIMDs of a CU busy
// rather than one; at the end the odd wave's lists go through LDS into the even wave's.
template <int DP, int KL, bool L2, int MODE, bool RS = false>
__global__ void __launch_bounds__(kThreads) flat_scan_kernel(ScanArgs a) {
  static_assert(!RS || 4 * 64 * KL <= kQueueCap * kThreads, "row-split hand-off must fit the queue arrays");
  if (gate_closed(a.gate, a.gate_want)) return;  // the same for every thread of the grid
  constexpr bool FILTER = MODE == 1;
  constexpr int H = DP / 2;                   // dims per lane half (K split in two halves)
  // LDS row stride in floats: conflict-free b128 reads. Columns DP and DP + 1 of a row hold the
  // augmented operand (||x||^2, 1) for L2, (1, 1) for the inner product.
  constexpr int STRIDE = DP + 4;
  constexpr int C4 = DP / 4;                  // float4 chunks per row
  constexpr int CHUNKS = kTileRows * C4;
  constexpr int PER_THREAD = (CHUNKS + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) float s_tile[2][kTileRows * STRIDE];
  __shared__ uint64_t s_bits[2];
  // Per-lane candidate queues, entry-major (entry e of thread t at e * kThreads + t) so lanes
  // appending at different depths never share a bank.
  __shared__ float s_qd[kQueueCap * kThreads];
  __shared__ uint32_t s_qr[kQueueCap * kThreads];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  // Workgroup w runs on XCD w % 8; give each XCD its own row splits so the workgroups resident
  // on one XCD at a time stream the same base rows through that XCD's L2.
  uint32_t qb, split;
  const uint32_t wg = blockIdx.x;
  if (a.nsplit % 8 == 0) {
    const uint32_t x = wg % 8, li = wg / 8;
    split = (li / a.qblocks) * 8 + x;
    qb = li % a.qblocks;
  } else {
    split = wg / a.qblocks;
    qb = wg % a.qblocks;
  }

  constexpr int kQPB = RS ? kQueriesPerBlock / 2 : kQueriesPerBlock;
  const int qgroup = RS ? (wave >> 1) : wave;  // the wave's 32 queries
  const int rb = RS ? (wave & 1) : 0;          // RS: the wave's 32-row half of each tile
  const uint32_t q = qb * kQPB + qgroup * 32 + j;
  const bool wave_active = qb * kQPB + qgroup * 32 < a.nq;
  const bool qvalid = q < a.nq;

  // This lane's half of its query: dims [h*H, h*H + H). MFMA step s pairs dim h*H+s of the query
  // (B operand, lane = (k=h, col=j)) with the same dim of a base row (A operand, lane = (row j, k=h)).
  // The matrix unit produces the distance itself: the query enters scaled by -2 (L2) or -1 (inner
  // product), both exact, and one more step adds the augmented pair, row (||x||^2, 1) against
  // query (1, ||q||^2) for L2 and (1, 1) against (1, 0) for the inner product, so the accumulator
  // ends at ||x||^2 + ||q||^2 - 2<q,x> or 1 - <q,x>.
  constexpr float kScale = L2 ? -2.0f : -1.0f;
  float qreg[H];
  {
    const f32x4* qp = reinterpret_cast<const f32x4*>(a.Q + static_cast<size_t>(qvalid ? q : 0) * DP + h * H);
#pragma unroll
    for (int s = 0; s < H / 4; ++s) {
      const f32x4 v = qvalid ? qp[s] : f32x4{0.f, 0.f, 0.f, 0.f};
      qreg[4 * s + 0] = kScale * v[0];
      qreg[4 * s + 1] = kScale * v[1];
      qreg[4 * s + 2] = kScale * v[2];
      qreg[4 * s + 3] = kScale * v[3];
    }
  }
  const float qaug = h == 0 ? 1.0f : (L2 && qvalid ? a.qnorm[q] : 0.0f);

  float Ld[KL];
  uint32_t Lr[KL];
#pragma unroll
  for (int x = 0; x < KL; ++x) {
    Ld[x] = __builtin_huge_valf();
    Lr[x] = QVH_EMPTY_ROW;
  }

  // Prune threshold: the smaller of this lane's KL-th best and the shared per-query value. Any
  // list's KL-th best bounds the KL-th best of the union of all lists, so candidates above it can
  // never be among the query's KL best (equal distances pass: ties are decided by row).
  uint32_t* const qw = a.qthr + static_cast<size_t>(qvalid ? q : 0u) * kScanBoundStride;
  float pthr = qvalid ? ordered_to_float(qw[0]) : __builtin_huge_valf();
  // Bound slots: every list of the query (one per split, row half rb and lane half h) publishes
  // its best distance, atomic min, to slot src of kScanSlots. A slot holds one row's distance at
  // any time, and different slots come from different lists, which hold different rows, so the
  // KL-th smallest slot value is at or above the query's KL-th best distance (KL distinct rows lie
  // at or below it); unwritten slots hold +inf. Slots read stale are larger, still bounds. With
  // many splits running at once this bound falls long before any one list holds KL good rows.
  static_assert(KL <= kScanSlots && kScanSlotBase + kScanSlots <= kScanBoundStride, "a query's slots fit its words");
  const uint32_t src =
      (split * (RS ? 4u : 2u) + static_cast<uint32_t>(rb) * 2u + static_cast<uint32_t>(h)) % kScanSlots;
  float published = __builtin_huge_valf();
  auto share_threshold = [&]() {
    // The two lanes of a query hold disjoint rows: their union has KL candidates at or below
    // max(own[KL/2-1], other[KL/2-1]) as well as below either list's KL-th.
    const float own_k = Ld[KL - 1], own_h = Ld[KL / 2 - 1];
    const float oth_k = __shfl_xor(own_k, 32, 64), oth_h = __shfl_xor(own_h, 32, 64);
    float t = fminf(fminf(own_k, oth_k), fmaxf(own_h, oth_h));
    if (a.share_rank != 0) {
      // k above KL (the wide merge): the pair's union has 2c >= R rows at or below the larger of
      // the two lanes' c-th entries.
      float own_c = Ld[0];
#pragma unroll
      for (int x = 1; x < KL; ++x) own_c = static_cast<uint32_t>(x) + 1 == a.share_rank ? Ld[x] : own_c;
      t = fmaxf(own_c, __shfl_xor(own_c, 32, 64));
    }
    if (qvalid) {
      uint32_t g = 0;
      if (h == 0) g = atomicMin(qw, float_to_ordered(t));
      uint32_t m = 0xFF800000u;  // +inf
      if (a.bound_slots) {
        if (Ld[0] < published) {
          published = Ld[0];
          __hip_atomic_fetch_min(qw + kScanSlotBase + src, float_to_ordered(published), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
        }
        // Each lane half reads half of the slots (ordered bits compare as the distances do) and
        // sorts them; the pair then takes the KL-th smallest of all kScanSlots.
        constexpr int kHalf = kScanSlots / 2;
        uint32_t sv[kHalf];
        uint64_t* sw = reinterpret_cast<uint64_t*>(qw + kScanSlotBase + h * kHalf);
#pragma unroll
        for (int i = 0; i < kHalf / 2; ++i) {
          const uint64_t w = __hip_atomic_load(sw + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          sv[2 * i] = static_cast<uint32_t>(w);
          sv[2 * i + 1] = static_cast<uint32_t>(w >> 32);
        }
        m = pair_kth_smallest<KL>(sv);
      }
      g = __shfl(g, j, 64);
      t = fminf(t, fminf(ordered_to_float(g), ordered_to_float(m)));
    }
    pthr = fminf(pthr, t);
  };

  // Candidate queue of this lane: appended in row order, inserted into the list by a wave-wide
  // flush (all lanes at once) when any queue could overflow on the next block.
  int qcount = 0;
  auto flush_queue = [&]() {
    int m = qcount;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
    for (int e = 0; e < m; ++e) {
      if (e < qcount) {
        float v = s_qd[e * kThreads + tid];
        v = v == v ? v : __builtin_huge_valf();
        if (v <= Ld[KL - 1]) list_insert_ordered<KL>(Ld, Lr, v, s_qr[e * kThreads + tid]);
      }
    }
    qcount = 0;
  };

  const uint64_t r0 = static_cast<uint64_t>(split) * a.rows_per_split;
  const uint64_t r1 = r0 < a.n ? (a.n < r0 + a.rows_per_split ? a.n : r0 + a.rows_per_split) : r0;
  const uint32_t ntiles = static_cast<uint32_t>(ceil_div(r1 - r0, kTileRows));

  f32x4 stage[PER_THREAD];
  float stage_norm = 0.0f;
  uint64_t stage_bits = ~0ull;
  // Unconditional loads (rows past the split repeat its last row; the epilogue masks them), so no
  // load sits under an exec-mask branch and the prefetch of the next tile stays in flight while
  // this tile's MFMAs run.
  const uint64_t last_row = r1 > r0 ? r1 - 1 : r0;
  auto load_tile = [&](uint32_t t) {
    const uint64_t base = r0 + static_cast<uint64_t>(t) * kTileRows;
#pragma unroll
    for (int p = 0; p < PER_THREAD; ++p) {
      int c = tid + p * kThreads;
      if (CHUNKS % kThreads != 0) c = c < CHUNKS ? c : CHUNKS - 1;
      const int row = c / C4, col = c % C4;
      uint64_t gr = base + row;
      gr = gr < last_row ? gr : last_row;
      stage[p] = *reinterpret_cast<const f32x4*>(a.X + gr * DP + 4 * col);
    }
    if constexpr (L2) {
      uint64_t gn = base + (tid & (kTileRows - 1));
      gn = gn < last_row ? gn : last_row;
      stage_norm = a.xnorm[gn];
    }
    if constexpr (FILTER) stage_bits = a.bitmap[base >> 6];
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PER_THREAD; ++p) {
      const int c = tid + p * kThreads;
      if (c < CHUNKS) {
        const int row = c / C4, col = c % C4;
        *reinterpret_cast<f32x4*>(&s_tile[buf][row * STRIDE + 4 * col]) = stage[p];
      }
    }
    if (tid < kTileRows) {
      *reinterpret_cast<f32x2*>(&s_tile[buf][tid * STRIDE + DP]) = f32x2{L2 ? stage_norm : 1.0f, 1.0f};
    }
    if (FILTER && tid == kTileRows) s_bits[buf] = stage_bits;
  };

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (uint32_t t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool prefetch = t + 1 < ntiles;
    if (!wave_active && prefetch) load_tile(t + 1);
    if (wave_active && RS) {
      // One 32-row half per wave: a single accumulation chain, four MFMAs per pair of b128 reads.
      f32x16 acc = {};
      const float* ar = &s_tile[buf][(32 * rb + j) * STRIDE + h * H];
      const float augr = s_tile[buf][(32 * rb + j) * STRIDE + DP + h];
      f32x4 x0 = *reinterpret_cast<const f32x4*>(ar);
#pragma unroll
      for (int s = 0; s < H; s += 4) {
        f32x4 n0 = x0;
        if (s + 4 < H) n0 = *reinterpret_cast<const f32x4*>(ar + s + 4);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[0], qreg[s + 0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[1], qreg[s + 1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[2], qreg[s + 2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[3], qreg[s + 3], acc, 0, 0, 0);
        x0 = n0;
        __builtin_amdgcn_sched_barrier(0);
        if (s == 4 && prefetch) load_tile(t + 1);
        if (s == 4) __builtin_amdgcn_sched_barrier(0);
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(augr, qaug, acc, 0, 0, 0);
      const uint64_t tile_row0 = r0 + static_cast<uint64_t>(t) * kTileRows;
      const uint64_t left = r1 - tile_row0;
      uint64_t admit = FILTER ? s_bits[buf] : ~0ull;
      if (left < 64) admit &= (1ull << left) - 1;
      const bool masked = FILTER || left < 64;
      const uint32_t lane_bits = static_cast<uint32_t>(admit >> (32 * rb)) >> (4 * h);
      const float thr = fminf(pthr, Ld[KL - 1]);
      bool any = false;
      if (!masked) {
        float m = acc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) m = fminf(m, acc[r]);
        any = !(m > thr);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) any = any || (!(acc[r] > thr) && ((lane_bits >> (8 * (r >> 2) + (r & 3))) & 1u));
      }
      any = any && qvalid;
      if (__builtin_amdgcn_ballot_w64(any)) {
        if (__builtin_amdgcn_ballot_w64(qcount > kQueueCap - 16)) flush_queue();
        const uint32_t row0 = static_cast<uint32_t>(tile_row0 + 32 * rb + 4 * h);
        if (masked) {
          queue_block<true>(acc, thr, any, lane_bits, row0, tid, qcount, s_qd, s_qr);
        } else {
          queue_block<false>(acc, thr, any, lane_bits, row0, tid, qcount, s_qd, s_qr);
        }
      }
    } else if (wave_active) {
      f32x16 acc0 = {}, acc1 = {};
      const float* a0 = &s_tile[buf][j * STRIDE + h * H];
      const float* a1 = &s_tile[buf][(32 + j) * STRIDE + h * H];
      // The augmented step's row operands (column DP + h), read first so they are in registers
      // by the end of the chain.
      const float aug0 = s_tile[buf][j * STRIDE + DP + h];
      const float aug1 = s_tile[buf][(32 + j) * STRIDE + DP + h];
      // Software-pipelined: the next step's two b128 LDS reads are issued before this step's
      // eight MFMAs (8 x 64 cycles), and the scheduling barrier keeps the compiler from hoisting
      // every read of the tile at once (which would spill).
      f32x4 x0 = *reinterpret_cast<const f32x4*>(a0);
      f32x4 x1 = *reinterpret_cast<const f32x4*>(a1);
#pragma unroll
      for (int s = 0; s < H; s += 4) {
        f32x4 n0 = x0, n1 = x1;
        if (s + 4 < H) {
          n0 = *reinterpret_cast<const f32x4*>(a0 + s + 4);
          n1 = *reinterpret_cast<const f32x4*>(a1 + s + 4);
        }
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[0], qreg[s + 0], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[0], qreg[s + 0], acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[1], qreg[s + 1], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[1], qreg[s + 1], acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[2], qreg[s + 2], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[2], qreg[s + 2], acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[3], qreg[s + 3], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[3], qreg[s + 3], acc1, 0, 0, 0);
        x0 = n0;
        x1 = n1;
        __builtin_amdgcn_sched_barrier(0);
        // The next tile's global loads go out once the MFMA pipe is busy, so no wait for them
        // lands in front of this tile's first MFMAs.
        if (s == 4 && prefetch) load_tile(t + 1);
        if (s == 4) __builtin_amdgcn_sched_barrier(0);
      }
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(aug0, qaug, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(aug1, qaug, acc1, 0, 0, 0);
      // D[row][col] of a 32x32 block: col = lane % 32 (query j), row = 8*(r/4) + 4*h + r%4 in
      // register r. Per lane the rows visited increase, so ties resolve to the smaller row.
      const uint64_t tile_row0 = r0 + static_cast<uint64_t>(t) * kTileRows;
      const uint64_t left = r1 - tile_row0;  // rows of this tile inside the split
      // Admitted rows of the tile (bit i = row tile_row0 + i), shifted to this lane half.
      uint64_t admit = FILTER ? s_bits[buf] : ~0ull;
      if (left < 64) admit &= (1ull << left) - 1;
      const bool masked = FILTER || left < 64;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        const f32x16 acc = blk ? acc1 : acc0;
        const uint32_t lane_bits = static_cast<uint32_t>(admit >> (32 * blk)) >> (4 * h);
        // Pass test: !(d > thr). Ties pass (a tied row may still win on row number), and so
        // does NaN, which the flush turns into +inf as the reference does.
        const float thr = fminf(pthr, Ld[KL - 1]);
        float d[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = acc[r];
        bool any = false;
        if (!masked) {  // wave-uniform: full tile, no filter
          // One test of the smallest distance (fminf skips NaN; all-NaN gives NaN, which passes).
          float m = d[0];
#pragma unroll
          for (int r = 1; r < 16; ++r) m = fminf(m, d[r]);
          any = !(m > thr);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            any = any || (!(d[r] > thr) && ((lane_bits >> (8 * (r >> 2) + (r & 3))) & 1u));
          }
        }
        // Lanes past the last query never queue: their zero query makes every inner-product
        // distance 1 exactly, a tie with their own list that would admit every row.
        any = any && qvalid;
        // Slow path: append this lane's passing, admitted candidates to its queue.
        if (__builtin_amdgcn_ballot_w64(any)) {
          if (__builtin_amdgcn_ballot_w64(qcount > kQueueCap - 16)) flush_queue();
          const uint32_t row0 = static_cast<uint32_t>(tile_row0 + 32 * blk + 4 * h);
          if (masked) {
            queue_block<true>(acc, thr, any, lane_bits, row0, tid, qcount, s_qd, s_qr);
          } else {
            queue_block<false>(acc, thr, any, lane_bits, row0, tid, qcount, s_qd, s_qr);
          }
        }
      }
    }
    if (wave_active && scan_share_after(t)) {
      flush_queue();
      if (a.share) share_threshold();
    }
    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (wave_active) flush_queue();
  if constexpr (RS) {
    // The odd wave of each query group hands its lists (rows of the tiles' second halves) to the
    // even wave through the queue arrays, free once every wave has flushed.
    __syncthreads();
    const int slot = (qgroup * 64 + lane) * KL;  // < 4 * 64 * KL <= kQueueCap * kThreads
    if (rb == 1) {
#pragma unroll
      for (int x = 0; x < KL; ++x) {
        s_qd[slot + x] = Ld[x];
        s_qr[slot + x] = Lr[x];
      }
    }
    __syncthreads();
    if (rb == 0) {
#pragma unroll
      for (int x = 0; x < KL; ++x) {
        const float d = s_qd[slot + x];
        if (d <= Ld[KL - 1]) list_insert<KL>(Ld, Lr, d, s_qr[slot + x]);
      }
    }
  }
  if (qvalid && rb == 0) {
    const size_t o = (static_cast<size_t>(q) * (2 * a.nsplit) + 2 * split + h) * KL;
#pragma unroll
    for (int x = 0; x < KL; ++x) {
      a.part_d[o + x] = Ld[x];
      a.part_r[o + x] = Lr[x];
    }
  }
}

// ---- the ring scan: small unfiltered batches -------------------------------------------------
//
// At most 32 queries are one 32-query group, which leaves the MFMA scan's 256-query blocks one wave
// in eight (or two in eight in its row-split form) and a single 64-row tile in flight per CU. Here
// each work-group is a row split and each of its four waves (one per SIMD) streams every fourth
// 32-row block of the split through a ring of LDS slots of its own. A slot holds one quarter of a
// block (32 rows x 32 dims), filled by direct global-to-LDS loads (global_load_lds_dwordx4, 16
// bytes per lane) several slots ahead of the MFMAs. Those loads are issued from inline assembly and
// waited for with explicit vmcnt counts: the compiler's own wait insertion would wait for every
// ring load in flight before each LDS read and drain the ring. The streaming loop issues no other
// vector memory instruction, so vmcnt counts exactly the ring's loads, which complete in issue
// order. Each slot's next quarter is read into registers while the current one's MFMAs run.
//
// Slot layout: lane i of load m writes 16-byte unit P = 64 m + i, which holds row P / 8 and the
// quarter's float4 column (P % 8) ^ (row % 8). MFMA lane (j, h) reads row j, columns 2u + h for
// u = 0..3, eight lanes of a read touching eight different columns (no bank conflicts).
//
// Distances are the MFMA scan's GEMM form: step t of quarter qq pairs dim 32 qq + 8 (t / 4) + 4 h
// + t % 4 of row j (A, lane (j, h)) with the same dim of query j scaled by -2 or -1 (B), and each
// block starts with the augmented step (||x||^2, 1) x (1, ||q||^2), or (1, 1) x (1, 0). The four
// waves keep per-lane lists and queues as the MFMA scan does and share a per-query bound through
// LDS and, across splits, through a per-query word in device memory; at the end their lists are
// merged into the first wave's, which writes two lists per query and split in the MFMA scan's
// format for the same merge, re-score and certificate.

constexpr int kRingWaves = 8;           // two per SIMD: one's selection runs beside the other's MFMAs
constexpr int kRingThreads = kRingWaves * 64;
constexpr int kRingSlots = 4;           // quarter-block slots per wave
constexpr int kRingSlotFloats = 32 * 32;
constexpr int kRingShareEvery = 2;      // blocks between exchanges of the shared bound
constexpr int kRingEarlyShares = 4;     // exchanges after each of a wave's first blocks
// With one wave per SIMD the next quarter is read into registers while this one's MFMAs run; with
// two, the other wave covers that read, and waiting for the next quarter only after the MFMAs
// keeps one more group of loads in flight meanwhile.
constexpr bool kRingLateWait = kRingWaves > 4;
constexpr uint32_t kRingMinQueries = 4;   // up to three queries the few-query kernel is faster
constexpr uint32_t kRingMaxQueries = 32;
constexpr uint64_t kRingMinSplitRows = 1024;  // rows per split at least (eight blocks per wave)
constexpr uint32_t kRingMaxSplits = 256;   // two lists per query and split: the merge's 512
constexpr uint32_t kRingBoundStride = 32;  // words between queries' bound slots (one 128-byte line each)

/// LDS byte address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}

/// One direct global-to-LDS load: lane i's 16 bytes at sbase + voff go to LDS address lds + 16 i.
/// M0 carries the LDS address for the load and gets its old value back afterwards. Vector memory
/// instructions other than these loads (the shared bound's atomic, which returns nothing) may only
/// make the explicit waits below wait longer: loads complete in issue order.
__device__ __forceinline__ void lds_load16(uint32_t lds, const void* sbase, uint32_t voff) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "s"(lds), "v"(voff), "s"(sbase)
      : "memory");
}

/// 4 bytes per lane from a per-lane address (lane i's to lds + 4 i).
__device__ __forceinline__ void lds_load4(uint32_t lds, const void* addr) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "s"(lds), "v"(addr)
      : "memory");
}

/// The bound slot that wave `wave`'s load for block b brings (the waves of a work-group and its
/// successive blocks go round the ns slots).
__device__ __forceinline__ uint32_t ring_slot_of(uint32_t b, int wave, int ns) {
  return (b * static_cast<uint32_t>(kRingWaves) + static_cast<uint32_t>(wave)) % static_cast<uint32_t>(ns);
}

/// Waits until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N <= 63, "vmcnt holds 0..63");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

/// wait_vmem<n>() for n in [LO, HI]; a constant n (an unrolled loop's) folds to the one wait.
template <int LO, int HI>
__device__ __forceinline__ void wait_vmem_n(int n) {
  if constexpr (LO <= HI) {
    if (n == LO) {
      wait_vmem<LO>();
    } else {
      wait_vmem_n<LO + 1, HI>(n);
    }
  }
}

/// Ring loads in the group of quarter qq of a block: four for the quarter's rows, and with quarter
/// 0 one more for the block's row norms and the queries' shared bounds.
__host__ __device__ constexpr int ring_group_loads(int qq) { return 4 + (qq == 0 ? 1 : 0); }

/// Loads that may still be outstanding once the group after quarter qq's has landed, the refill of
/// quarter qq + R - 1 having just been issued: those of the R - 2 groups issued after that group
/// (quarters qq + 2 .. qq + R - 1, modulo NQ).
template <int NQ>
__host__ __device__ constexpr int ring_wait_count(int qq) {
  int n = 0;
  for (int d = 2; d <= kRingSlots - 1; ++d) n += ring_group_loads((qq + d) % NQ);
  return n;
}

/// The value of lane (lane ^ 32), by one v_permlane32_swap (no LDS round trip).
__device__ __forceinline__ uint32_t lane_swap32_u32(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}
__device__ __forceinline__ float lane_swap32_f(float v) { return __uint_as_float(lane_swap32_u32(__float_as_uint(v))); }

/// The key of an empty list entry: +inf distance, QVH_EMPTY_ROW (after every real entry).
constexpr uint64_t kRingEmptyKey = (uint64_t{0xFF800000u} << 32) | QVH_EMPTY_ROW;

/// Inserts `key` into the ascending (distance, row) key list K, dropping the last entry. Every entry
/// takes one compare and two selects, none waiting on another's (the list is sorted, so the
/// entries above the key form a suffix that shifts up by one); the empty key changes nothing.
template <int KL>
__device__ __forceinline__ void key_insert(uint64_t (&K)[KL], uint64_t key) {
  bool gt[KL];
#pragma unroll
  for (int x = 0; x < KL; ++x) gt[x] = K[x] > key;
#pragma unroll
  for (int x = KL - 1; x > 0; --x) K[x] = gt[x] ? (gt[x - 1] ? K[x - 1] : key) : K[x];
  K[0] = gt[0] ? key : K[0];
}

/// Sorts 16 keys ascending in registers (a bitonic network, 80 compare-exchanges).
__device__ __forceinline__ void sort16_keys(uint64_t (&k)[16]) {
#pragma unroll
  for (int w = 2; w <= 16; w <<= 1) {
#pragma unroll
    for (int s = w >> 1; s > 0; s >>= 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int l = i ^ s;
        if (l > i) {
          const bool up = (i & w) == 0;
          const uint64_t x = k[i], y = k[l];
          const bool sw = up ? (x > y) : (x < y);
          k[i] = sw ? y : x;
          k[l] = sw ? x : y;
        }
      }
    }
  }
}

/// Distance of a (distance, row) key.
__device__ __forceinline__ float key_distance(uint64_t k) { return ordered_to_float(static_cast<uint32_t>(k >> 32)); }

/// Merges the sorted key list at sk (entry x of this lane at x * 64 + lane) into K: the KL best of
/// the union. An entry that would not enter ends the lane's part (every later one is after it),
/// and the wave stops once no lane takes one.
template <int KL>
__device__ __forceinline__ void ring_merge_list(uint64_t (&K)[KL], const uint64_t* sk, int lane) {
  for (int x = 0; x < KL; ++x) {
    const uint64_t k = sk[x * 64 + lane];
    const bool take = k < K[KL - 1];
    if (!__builtin_amdgcn_ballot_w64(take)) break;
    key_insert<KL>(K, take ? k : kRingEmptyKey);
  }
}

template <int DP, int KL, bool L2>
__global__ void __launch_bounds__(kRingThreads) flat_ring_kernel(ScanArgs a) {
  static_assert(DP % 32 == 0 && DP <= kMaxDp, "the ring scan takes whole 32-dim quarters");
  static_assert(kRingWaves / 2 * KL * 64 * 2 <= kRingWaves * kRingSlots * kRingSlotFloats, "list hand-off fits the rings");
  static_assert((kRingWaves & (kRingWaves - 1)) == 0 && kRingWaves >= 2, "the hand-off halves the waves");
  if (gate_closed(a.gate, a.gate_want)) return;  // the same for every thread of the grid
  constexpr int NQ = DP / 32;  // quarters per block
  constexpr int R = kRingSlots;
  constexpr int SLOT_BYTES = kRingSlotFloats * 4;
  __shared__ __attribute__((aligned(16))) float s_ring[kRingWaves][R][kRingSlotFloats];
  __shared__ float s_norm[kRingWaves][R][64];
  __shared__ uint32_t s_thr[32];
  // Per query, the ceil(KL / NL)-th entry of each of the work-group's NL lists (two lane halves
  // per wave, disjoint rows): their union holds KL entries at or below the largest.
  constexpr int NL = 2 * kRingWaves;
  __shared__ __attribute__((aligned(16))) float s_part[32][NL];
  // Per query, NS bound slots in device memory (a.qthr, kRingBoundStride words per query): slot s
  // holds the smallest distance any split of class s (split % NS) has found, so the NS slots are
  // distances of NS different rows and their largest bounds the KL-th (NS >= KL). Each block's
  // norm load brings one slot of each query (rotating over the slots); s_slot keeps the smallest
  // value seen per slot, and the work-group's best distance goes to its own slot.
  constexpr int NS = KL <= 16 ? 16 : 32;
  static_assert(NS <= static_cast<int>(kRingBoundStride), "the slots fit a query's line");
  __shared__ __attribute__((aligned(16))) uint32_t s_slot[32][NS];
  __shared__ uint32_t s_best[32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, h = lane >> 5;
  const uint32_t split = blockIdx.x;
  const uint32_t q = static_cast<uint32_t>(j);
  const bool qvalid = q < a.nq;

  // This split's rows (the grid has no empty split) and this wave's blocks: wave, wave + 4, ...
  const uint64_t r0 = static_cast<uint64_t>(split) * a.rows_per_split;
  const uint64_t r1 = a.n < r0 + a.rows_per_split ? a.n : r0 + a.rows_per_split;
  const uint32_t nblk = static_cast<uint32_t>(ceil_div(r1 - r0, 32));
  const uint32_t myblk = nblk > static_cast<uint32_t>(wave) ? (nblk - wave + kRingWaves - 1) / kRingWaves : 0u;

  constexpr float kScale = L2 ? -2.0f : -1.0f;
  float qreg[DP / 2];
  {
    const float* qp = a.Q + static_cast<size_t>(qvalid ? q : 0) * DP;
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4 v = qvalid ? *reinterpret_cast<const f32x4*>(qp + 32 * qq + 8 * u + 4 * h)
                               : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) qreg[qq * 16 + 4 * u + i] = kScale * v[i];
      }
  }
  const float qaug = h == 0 ? 1.0f : (L2 && qvalid ? a.qnorm[q] : 0.0f);
  // Uses that make the compiler wait for these loads here, before any ring load is in flight.
#pragma unroll
  for (int i = 0; i < DP / 2; ++i) asm volatile("" ::"v"(qreg[i]));
  asm volatile("" ::"v"(qaug));

  if (tid < 32) s_thr[tid] = 0xFF800000u;  // ordered bits of +inf
  for (int i = tid; i < 32 * NL; i += kRingThreads) s_part[i / NL][i % NL] = __builtin_huge_valf();
  for (int i = tid; i < 32 * NS; i += kRingThreads) s_slot[i / NS][i % NS] = 0xFF800000u;
  if (tid < 32) s_best[tid] = 0xFF800000u;
  __syncthreads();

  uint64_t Lk[KL];  // this lane's list: the KL best (distance, row) keys of its rows, ascending
#pragma unroll
  for (int x = 0; x < KL; ++x) Lk[x] = kRingEmptyKey;
  float pthr = __builtin_huge_valf();

  if (myblk > 0) {
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(&s_ring[wave][0][0]));
    const uint32_t norm_lds = __builtin_amdgcn_readfirstlane(lds_address(&s_norm[wave][0][0]));
    const float* ring = &s_ring[wave][0][0];
    const float* norms = &s_norm[wave][0][0];
    // Byte offsets of this lane's 16-byte units in a whole block's quarter, and of its row norm.
    uint32_t voff[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t P = 64 * m + lane, r = P >> 3, c = (P & 7) ^ (r & 7);
      voff[m] = (r * DP + 4 * c) * 4;
    }
    // Quarter qq of block b (clamped to the wave's last block: the loads past the end repeat it,
    // so every group has its fixed number of loads) into slot `slot`, once every LDS read this
    // wave has issued is complete (among them the last reads of that slot).
    auto issue = [&](uint32_t b, int qq, uint32_t slot) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const uint32_t b_virtual = b;
      b = b < myblk ? b : myblk - 1;
      const uint64_t row0 = r0 + 32ull * (static_cast<uint64_t>(wave) + kRingWaves * static_cast<uint64_t>(b));
      const uint64_t left = r1 - row0;  // >= 1
      const float* sbase = a.X + row0 * DP + 32 * qq;
      const uint32_t lds = ring_lds + slot * SLOT_BYTES;
      if (left >= 32) {
#pragma unroll
        for (int m = 0; m < 4; ++m) lds_load16(lds + 1024 * m, sbase, voff[m]);
      } else {  // the split's last block: rows past its end repeat its last row
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint32_t P = 64 * m + lane, r = P >> 3, c = (P & 7) ^ (r & 7);
          const uint32_t rc = r < left ? r : static_cast<uint32_t>(left - 1);
          lds_load16(lds + 1024 * m, sbase, (rc * DP + 4 * c) * 4);
        }
      }
      if (qq == 0) {  // lanes 0-31: the block's row norms (L2); 32-63: one bound slot per query
        const uint32_t rn = static_cast<uint32_t>(j) < left ? static_cast<uint32_t>(j) : static_cast<uint32_t>(left - 1);
        const void* src = L2 && h == 0 ? static_cast<const void*>(a.xnorm + row0 + rn)
                                       : static_cast<const void*>(a.qthr + (qvalid ? q : 0u) * kRingBoundStride +
                                                                  ring_slot_of(b_virtual, wave, NS));
        lds_load4(norm_lds + slot * 256, src);
      }
    };
    auto read = [&](uint32_t slot, f32x4 (&x)[4]) {
      const float* sp = ring + slot * kRingSlotFloats;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = 2 * u + h;
        x[u] = *reinterpret_cast<const f32x4*>(sp + (j * 8 + (c ^ (j & 7))) * 4);
      }
    };

    // Prologue: groups 0 .. R - 2 in flight, then group 0 in registers.
#pragma unroll
    for (int g = 0; g < R - 1; ++g) issue(static_cast<uint32_t>(g / NQ), g % NQ, static_cast<uint32_t>(g));
    uint32_t slot_read = 0, slot_issue = R - 1;
    {
      constexpr int kFirst = [] {
        int n = 0;
        for (int d = 1; d <= kRingSlots - 2; ++d) n += ring_group_loads(d % NQ);
        return n;
      }();
      wait_vmem<kFirst>();
    }
    f32x4 xa[4], xb[4];
    read(0, xa);
    float na = L2 ? norms[j] : 1.0f, nb = na;
    uint32_t ga = __float_as_uint(norms[32 + j]), gb = ga;  // the block's bound slot as its load saw it

    for (uint32_t b = 0; b < myblk; ++b) {
      f32x16 acc = {};
#pragma unroll
      for (int qq = 0; qq < NQ; ++qq) {
        if (qq == 0) {
          acc = __builtin_amdgcn_mfma_f32_32x32x2f32(h == 0 ? na : 1.0f, qaug, acc, 0, 0, 0);
          if (h == 0) atomicMin(&s_slot[j][ring_slot_of(b, wave, NS)], ga);
        }
        // Refill the slot this quarter's predecessor used (read in the iteration before last), then
        // wait for the next group and read it while this quarter's MFMAs run.
        issue(b + (qq + R - 1) / NQ, (qq + R - 1) % NQ, slot_issue);
        slot_issue = slot_issue + 1 == R ? 0 : slot_issue + 1;
        const uint32_t slot_next = slot_read + 1 == R ? 0 : slot_read + 1;
        auto next = [&]() {
          wait_vmem_n<4 * (kRingSlots - 2), 5 * (kRingSlots - 2)>(ring_wait_count<NQ>(qq));
          read(slot_next, xb);
          if ((qq + 1) % NQ == 0) {
            if (L2) nb = norms[slot_next * 64 + j];
            gb = __float_as_uint(norms[slot_next * 64 + 32 + j]);
          }
        };
        if (!kRingLateWait) next();
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[u][i], qreg[qq * 16 + 4 * u + i], acc, 0, 0, 0);
        if (kRingLateWait) next();
#pragma unroll
        for (int u = 0; u < 4; ++u) xa[u] = xb[u];
        if ((qq + 1) % NQ == 0) {
          na = nb;
          ga = gb;
        }
        slot_read = slot_next;
      }
      // Selection over the block: register r holds row 8 (r / 4) + 4 h + r % 4 of the block.
      const uint64_t row0 = r0 + 32ull * (static_cast<uint64_t>(wave) + kRingWaves * static_cast<uint64_t>(b));
      const uint64_t left = r1 - row0;
      const bool masked = left < 32;
      const uint32_t lane_bits = (masked ? ((1u << left) - 1u) : 0xFFFFFFFFu) >> (4 * h);
      const float thr = fminf(pthr, key_distance(Lk[KL - 1]));
      bool any = false;
      if (!masked) {
        float m = acc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) m = fminf(m, acc[r]);
        any = !(m > thr);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) any = any || (!(acc[r] > thr) && ((lane_bits >> (8 * (r >> 2) + (r & 3))) & 1u));
      }
      any = any && qvalid;
      if (b == 0) {
        // The wave's first block, into empty lists: its 16 candidates sorted (NaN as +inf), the
        // KL smallest kept; rows that do not pass (outside the split) are empty keys.
        uint64_t k16[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int bit = 8 * (r >> 2) + (r & 3);
          const bool p = qvalid && (!masked || ((lane_bits >> bit) & 1u));
          const float v = acc[r] == acc[r] ? acc[r] : __builtin_huge_valf();
          k16[r] = p ? make_key(v, static_cast<uint32_t>(row0 + 4 * h + bit)) : kRingEmptyKey;
        }
        sort16_keys(k16);
#pragma unroll
        for (int x = 0; x < KL; ++x) Lk[x] = x < 16 ? k16[x < 16 ? x : 0] : kRingEmptyKey;
      } else if (__builtin_amdgcn_ballot_w64(any)) {
        // Passing candidates straight into the list (NaN as +inf), one register at a time across
        // the wave, for the registers where some lane has one (the other wave of the SIMD runs its
        // MFMAs meanwhile).
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int bit = 8 * (r >> 2) + (r & 3);
          bool p = any && !(acc[r] > thr);
          if (masked) p = p && ((lane_bits >> bit) & 1u);
          if (__builtin_amdgcn_ballot_w64(p)) {
            const float v = acc[r] == acc[r] ? acc[r] : __builtin_huge_valf();
            key_insert<KL>(Lk, p ? make_key(v, static_cast<uint32_t>(row0 + 4 * h + bit)) : kRingEmptyKey);
          }
        }
      }
      if (b < kRingEarlyShares || b % kRingShareEvery == kRingShareEvery - 1) {
        // The two lanes of a query hold disjoint rows, and so do the waves and the splits: any
        // list's KL-th (or the lane pair's bound, or the work-group's union bound, or the largest
        // bound slot) bounds the KL-th of the union of all of the query's lists; the smallest of
        // them goes to the work-group through LDS.
        const float own_k = key_distance(Lk[KL - 1]), own_h = key_distance(Lk[KL / 2 - 1]);
        const float oth_k = lane_swap32_f(own_k), oth_h = lane_swap32_f(own_h);
        float t = fminf(fminf(own_k, oth_k), fmaxf(own_h, oth_h));
        // The work-group's union: the other waves' entries may be older (larger) values of their
        // lists, which keeps the largest of the eight an upper bound.
        s_part[j][2 * wave + h] = key_distance(Lk[(KL + NL - 1) / NL - 1]);
        {
          float u = -__builtin_huge_valf();
#pragma unroll
          for (int c = 0; c < NL; c += 4) {
            const f32x4 pc = *reinterpret_cast<const f32x4*>(&s_part[j][c]);
            u = fmaxf(u, fmaxf(fmaxf(pc[0], pc[1]), fmaxf(pc[2], pc[3])));
          }
          t = fminf(t, u);
        }
        // The slots: the largest of the smallest values seen per slot.
        {
          uint32_t smax = 0u;
#pragma unroll
          for (int c = 0; c < NS; c += 4) {
            const uint32_t* sp = &s_slot[j][c];
            smax = max(smax, max(max(sp[0], sp[1]), max(sp[2], sp[3])));
          }
          t = fminf(t, ordered_to_float(smax));
        }
        // This work-group's best distance per query, into its slot when below the slot's value as
        // last seen here (an atomic that returns nothing: the ring's waits never wait for a return,
        // but may wait behind it, so these stay few).
        const uint32_t mine = float_to_ordered(key_distance(Lk[0]));
        uint32_t g = 0xFF800000u;
        if (h == 0) {
          const uint32_t ot = float_to_ordered(t);
          g = atomicMin(&s_thr[j], ot);
          const uint32_t best = atomicMin(&s_best[j], mine);
          const uint32_t wb = best < mine ? best : mine;
          const uint32_t own = split % NS;
          if (wave == 0 && qvalid && wb < s_slot[j][own]) {
            atomicMin(&s_slot[j][own], wb);
            __hip_atomic_fetch_min(a.qthr + q * kRingBoundStride + own, wb, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          }
        } else {
          atomicMin(&s_best[j], mine);
        }
        const uint32_t gs = lane_swap32_u32(g);
        g = h == 0 ? g : gs;
        pthr = fminf(pthr, fminf(t, ordered_to_float(g)));
      }
    }
    wait_vmem<0>();  // the loads past the end, before the LDS is reused or released
  }

  // The waves' lists into the first wave's, through the ring slots, halving the waves each round:
  // waves [s, 2s) hand theirs to waves [0, s).
  uint64_t* hk = reinterpret_cast<uint64_t*>(&s_ring[0][0][0]);
#pragma unroll
  for (int s = kRingWaves / 2; s >= 1; s /= 2) {
    __syncthreads();
    if (wave >= s && wave < 2 * s) {
#pragma unroll
      for (int x = 0; x < KL; ++x) hk[((wave - s) * KL + x) * 64 + lane] = Lk[x];
    }
    __syncthreads();
    if (wave < s) ring_merge_list<KL>(Lk, hk + wave * KL * 64, lane);
  }
  if (wave == 0) {
    if (qvalid) {
      const size_t o = (static_cast<size_t>(q) * (2 * a.nsplit) + 2 * split + h) * KL;
#pragma unroll
      for (int x = 0; x < KL; ++x) {
        a.part_d[o + x] = key_distance(Lk[x]);
        a.part_r[o + x] = static_cast<uint32_t>(Lk[x]);
      }
    }
  }
}

// ---- the chunked scan: rows wider than kMaxDp ------------------------------------------------
//
// The same search for any padded width: each step stages one kKc-dim chunk of a 64-row tile and of
// the block's 256 queries (scaled by -2 or -1 on the way in) in LDS, and every wave accumulates its
// 32 queries x 64 rows over the chunks; after a tile's last chunk the augmented step adds
// (||x||^2, 1) x (1, ||q||^2) and the tile goes through the same selection as the register scan.
// The next step's loads are in flight while a step's 32 MFMAs per wave run.
constexpr int kKc = 32;              // dims per chunk
constexpr int kKcStride = kKc + 4;   // LDS row stride of a row chunk (floats)
constexpr int kKcQueueCap = 18;      // queue entries per lane (LDS holds both chunk buffers too)
constexpr uint32_t kMaxChunkedDp = 4096;
// Largest contiguous copy of listed rows for the MFMA scan; a filter admitting more rows goes to
// the scan as its bitmap.
constexpr uint64_t kCompactMaxBytes = 4ull << 30;

template <int KL, bool L2, int MODE>
__global__ void __launch_bounds__(kThreads) flat_scan_k_kernel(ScanArgs a) {
  if (gate_closed(a.gate, a.gate_want)) return;  // the same for every thread of the grid
  constexpr bool FILTER = MODE == 1;
  constexpr int C4 = kKc / 4;  // float4 slots per chunk row
  __shared__ __attribute__((aligned(16))) float s_x[2][kTileRows * kKcStride];
  // Query chunks: slot (row, c) of row-major [256][C4] float4 slots at row * C4 + (c ^ (row % 8)),
  // so a wave's 32 rows reading one column spread over the banks.
  __shared__ __attribute__((aligned(16))) float s_q[2][kQueriesPerBlock * kKc];
  __shared__ float s_aug[2][kTileRows];
  __shared__ uint64_t s_bits[2];
  __shared__ float s_qd[kKcQueueCap * kThreads];
  __shared__ uint32_t s_qr[kKcQueueCap * kThreads];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  uint32_t qb, split;
  scan_block_coords(a, qb, split);
  const uint32_t q = qb * kQueriesPerBlock + wave * 32 + j;
  const bool wave_active = qb * kQueriesPerBlock + wave * 32 < a.nq;
  const bool qvalid = q < a.nq;
  constexpr float kScale = L2 ? -2.0f : -1.0f;
  const float qaug = h == 0 ? 1.0f : (L2 && qvalid ? a.qnorm[q] : 0.0f);

  LaneScan<KL, kKcQueueCap> ls;
  ls.init(tid, qvalid ? ordered_to_float(a.qthr[static_cast<size_t>(q) * kScanBoundStride]) : __builtin_huge_valf());

  const uint64_t r0 = static_cast<uint64_t>(split) * a.rows_per_split;
  const uint64_t r1 = r0 < a.n ? (a.n < r0 + a.rows_per_split ? a.n : r0 + a.rows_per_split) : r0;
  const uint32_t ntiles = static_cast<uint32_t>(ceil_div(r1 - r0, kTileRows));
  const uint32_t nchunks = (a.dp + kKc - 1) / kKc;
  const uint64_t nsteps = static_cast<uint64_t>(ntiles) * nchunks;
  const uint64_t last_row = r1 > r0 ? r1 - 1 : r0;

  // Staging registers: one row slot and four query slots per thread, and per tile the row norm
  // (threads 0-63) and the filter word (thread 64).
  const int xrow = tid / C4, xc = tid % C4;  // 64 rows x 8 slots = 512 = kThreads
  uint64_t xg = 0;                           // global row of xrow in the current tile
  f32x4 sx, sq[4];
  float sn = 0.0f;
  uint64_t sb = ~0ull;
  auto load_step = [&](uint64_t i) {
    const uint32_t t = static_cast<uint32_t>(i / nchunks), c = static_cast<uint32_t>(i % nchunks);
    const uint64_t base = r0 + static_cast<uint64_t>(t) * kTileRows;
    if (c == 0) {
      uint64_t gr = base + xrow;
      gr = gr < last_row ? gr : last_row;
      xg = gr;
      if (L2 && tid < kTileRows) {
        uint64_t gn = base + tid;
        gn = gn < last_row ? gn : last_row;
        sn = a.xnorm[gn];
      }
      if (FILTER && tid == kTileRows) sb = a.bitmap[base >> 6];
    }
    const uint32_t col = c * kKc + 4 * xc;
    sx = col < a.dp ? *reinterpret_cast<const f32x4*>(a.X + xg * a.dp + col) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int item = tid + p * kThreads, qr = item / C4, qc = item % C4;
      uint32_t qg = qb * kQueriesPerBlock + qr;
      qg = qg < a.nq ? qg : a.nq - 1;
      const uint32_t qcol = c * kKc + 4 * qc;
      sq[p] = qcol < a.dp ? *reinterpret_cast<const f32x4*>(a.Q + static_cast<uint64_t>(qg) * a.dp + qcol)
                          : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store_step = [&](uint64_t i, int buf) {
    const uint32_t t = static_cast<uint32_t>(i / nchunks), c = static_cast<uint32_t>(i % nchunks);
    *reinterpret_cast<f32x4*>(&s_x[buf][xrow * kKcStride + 4 * xc]) = sx;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int item = tid + p * kThreads, qr = item / C4, qc = item % C4;
      *reinterpret_cast<f32x4*>(&s_q[buf][4 * (qr * C4 + (qc ^ (qr % 8)))]) = kScale * sq[p];
    }
    if (c == 0) {
      if (tid < kTileRows) s_aug[t & 1][tid] = L2 ? sn : 1.0f;
      if (FILTER && tid == kTileRows) s_bits[t & 1] = sb;
    }
  };

  if (nsteps > 0) {
    load_step(0);
    store_step(0, 0);
  }
  __syncthreads();

  f32x16 acc0 = {}, acc1 = {};
  const int qrow = wave * 32 + j;
  for (uint64_t i = 0; i < nsteps; ++i) {
    const int buf = static_cast<int>(i & 1);
    const uint32_t t = static_cast<uint32_t>(i / nchunks), c = static_cast<uint32_t>(i % nchunks);
    const bool prefetch = i + 1 < nsteps;
    if (prefetch) load_step(i + 1);
    if (wave_active) {
      if (c == 0) {
        acc0 = f32x16{};
        acc1 = f32x16{};
      }
      // Lane (j, h): dims h*16 .. h*16+15 of the chunk, as four float4 slots.
      f32x4 b[4], x0[4], x1[4];
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int slot = h * 4 + s4;
        b[s4] = *reinterpret_cast<const f32x4*>(&s_q[buf][4 * (qrow * C4 + (slot ^ (qrow % 8)))]);
        x0[s4] = *reinterpret_cast<const f32x4*>(&s_x[buf][j * kKcStride + 4 * slot]);
        x1[s4] = *reinterpret_cast<const f32x4*>(&s_x[buf][(32 + j) * kKcStride + 4 * slot]);
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[s4][e], b[s4][e], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[s4][e], b[s4][e], acc1, 0, 0, 0);
        }
      }
      if (c + 1 == nchunks) {
        const float aug0 = h == 0 ? s_aug[t & 1][j] : 1.0f;
        const float aug1 = h == 0 ? s_aug[t & 1][32 + j] : 1.0f;
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(aug0, qaug, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(aug1, qaug, acc1, 0, 0, 0);
        const uint64_t tile_row0 = r0 + static_cast<uint64_t>(t) * kTileRows;
        ls.tile(acc0, acc1, tile_row0, r1 - tile_row0, FILTER ? s_bits[t & 1] : ~0ull, FILTER, qvalid, h, s_qd, s_qr);
        if ((t % kShareEvery) == kShareEvery - 1) {
          ls.flush(s_qd, s_qr);
          if (a.share) ls.share(qvalid ? &a.qthr[static_cast<size_t>(q) * kScanBoundStride] : nullptr, h, j);
        }
      }
    }
    if (prefetch) store_step(i + 1, buf ^ 1);
    __syncthreads();
  }

  if (wave_active) ls.flush(s_qd, s_qr);
  if (qvalid) ls.store(a.part_d, a.part_r, (static_cast<size_t>(q) * (2 * a.nsplit) + 2 * split + h) * KL);
}

struct MergeArgs {
  const float* X;
  uint32_t dim, dp;
  const float* Q;
  uint32_t nq, k;
  int l2;
  uint32_t nlists;          // 2 * nsplit
  const float* part_d;
  const uint32_t* part_r;
  const uint32_t* idx;  // list positions -> rows (indexed scan), or null
  uint32_t* out_rows;
  float* out_dist;
  const float* delta;   // [nq] bound on |GEMM-form distance - exact distance| (prep_queries_kernel)
  uint32_t* fallback;   // queries the exact kernel recomputes (uncertified selections)
  uint32_t* nfallback;  // their count
  const uint32_t* gate;  // as ScanArgs::gate
  uint32_t gate_want;
};

/// Certificate of a re-scored selection. The selection holds the `sel` best candidates by GEMM-form
/// distance, the last of which is g_last; every other admitted row has a GEMM-form distance of at
/// least g_last (the scan's bounds only drop rows above some list's sel-th distance, which is at
/// least the union's). An unselected row's exact distance is then at least g_last - delta, so when
/// the k-th smallest exact distance of the selection lies strictly below that, no unselected row can
/// enter the top k. A selection that took every admitted row (count < sel) is complete, and with
/// delta = 0 the two forms agree exactly, so the (distance, row) order of the selection is final.
__device__ __forceinline__ bool selection_certified(uint32_t count, uint32_t sel, float g_last, float e_k,
                                                    float delta) {
  if (count < sel || delta == 0.0f) return true;
  return static_cast<double>(e_k) < static_cast<double>(g_last) - static_cast<double>(delta);
}

/// Keys held per list by the merge before it reloads.
constexpr int kMergeHeld = 4;

/// Keys p .. p + kMergeHeld - 1 of one list (positions at or past KL read the list's start: in
/// bounds, never used), as 16-byte loads when KL keeps them aligned.
template <int KL>
__device__ __forceinline__ void merge_load_held(const float* ld, const uint32_t* lr, uint32_t p, float (&d)[kMergeHeld],
                                                uint32_t (&r)[kMergeHeld]) {
  static_assert(kMergeHeld == 4, "one 16-byte load per list");
  if constexpr (KL % 4 == 0) {
    const uint32_t at = p + 4 <= KL ? p : 0u;
    const f32x4 dv = *reinterpret_cast<const f32x4*>(ld + at);
    const f32x4 rv = *reinterpret_cast<const f32x4*>(lr + at);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d[i] = dv[i];
      r[i] = __float_as_uint(rv[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t at = p + i < KL ? p + i : 0u;
      d[i] = ld[at];
      r[i] = lr[at];
    }
  }
}

template <int KL>
__global__ void __launch_bounds__(256) flat_merge_kernel(MergeArgs m) {
  if (gate_closed(m.gate, m.gate_want)) return;
  const int lane = threadIdx.x & 63;
  const uint32_t q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= m.nq) return;  // whole wave; this kernel has no block barriers
  const float* pd = m.part_d + static_cast<size_t>(q) * m.nlists * KL;
  const uint32_t* pr = m.part_r + static_cast<size_t>(q) * m.nlists * KL;

  // The first kMergeHeld keys of each list are loaded up front (unconditional loads, clamped to a
  // list that exists, so none waits behind a branch) and popped from registers; a list whose held
  // keys run out before its KL-th loads its next ones there and then. The pop loop itself issues
  // no other memory access, so no pop waits for an earlier one's load.
  constexpr int H = kMergeHeld;
  uint64_t kk[kMaxListsPerLane][H];
  uint32_t ptr[kMaxListsPerLane];  // the position of kk[u][0] in list u
#pragma unroll
  for (int u = 0; u < kMaxListsPerLane; ++u) {
    const uint32_t li = lane + 64 * u;
    const bool ok = li < m.nlists;
    const uint32_t lc = ok ? li : 0u;
    float d[H];
    uint32_t r[H];
    merge_load_held<KL>(pd + static_cast<size_t>(lc) * KL, pr + static_cast<size_t>(lc) * KL, 0, d, r);
#pragma unroll
    for (int i = 0; i < H; ++i) kk[u][i] = ok && i < KL ? make_key(d[i], r[i]) : ~0ull;
    ptr[u] = 0;
  }
  uint64_t sel = ~0ull;
  int count = 0;
  for (int x = 0; x < KL; ++x) {
    uint64_t mine = kk[0][0];
    int arg = 0;
#pragma unroll
    for (int u = 1; u < kMaxListsPerLane; ++u) {
      if (kk[u][0] < mine) {
        mine = kk[u][0];
        arg = u;
      }
    }
    const uint64_t best = wave_min_u64(mine);
    if (static_cast<uint32_t>(best) == QVH_EMPTY_ROW) break;  // only empty slots remain
    if (lane == x) sel = best;
    ++count;
    if (mine == best) {
#pragma unroll
      for (int u = 0; u < kMaxListsPerLane; ++u) {
        if (u == arg) {
#pragma unroll
          for (int i = 0; i + 1 < H; ++i) kk[u][i] = kk[u][i + 1];
          kk[u][H - 1] = ~0ull;
          const uint32_t p = ++ptr[u];
          if (p % H == 0 && p < KL) {  // held keys used up: the list's next ones
            float d[H];
            uint32_t r[H];
            merge_load_held<KL>(pd + static_cast<size_t>(lane + 64 * u) * KL,
                                pr + static_cast<size_t>(lane + 64 * u) * KL, p, d, r);
#pragma unroll
            for (int i = 0; i < H; ++i) kk[u][i] = p + i < KL ? make_key(d[i], r[i]) : ~0ull;
          }
        }
      }
    }
  }
  // Re-score the selected candidates exactly and rank them by (distance, row).
  const bool valid = lane < count;
  const uint32_t row = valid && m.idx ? m.idx[static_cast<uint32_t>(sel)] : static_cast<uint32_t>(sel);
  float e = __builtin_huge_valf();
  if (valid) {
    e = exact_flat_distance(m.Q + static_cast<size_t>(q) * m.dp,
                            m.X + static_cast<size_t>(row) * m.dp, m.dim, m.l2 != 0);
  }
  const uint64_t key = valid ? make_key(e, row) : ~0ull;
  uint32_t rank = 0;
  for (int y = 0; y < KL; ++y) {
    const uint64_t o = __shfl(key, y, 64);
    rank += o < key ? 1u : 0u;
  }
  // The KL-th selected GEMM-form distance (lane KL - 1) and the k-th smallest exact distance.
  const float g_last = ordered_to_float(static_cast<uint32_t>(__shfl(sel, KL - 1, 64) >> 32));
  float e_k = valid && rank < m.k ? e : -__builtin_huge_valf();
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) e_k = fmaxf(e_k, __shfl_xor(e_k, off, 64));
  if (!selection_certified(static_cast<uint32_t>(count), KL, g_last, e_k, m.delta[q])) {
    if (lane == 0) m.fallback[atomicAdd(m.nfallback, 1u)] = q;
    return;
  }
  uint32_t* orow = m.out_rows + static_cast<size_t>(q) * m.k;
  float* odist = m.out_dist + static_cast<size_t>(q) * m.k;
  if (valid && rank < m.k) {
    orow[rank] = row;
    odist[rank] = e;
  }
  for (uint32_t p = lane; p < m.k; p += 64) {
    if (p >= static_cast<uint32_t>(count)) {
      orow[p] = QVH_EMPTY_ROW;
      odist[p] = __builtin_huge_valf();
    }
  }
}

// k from 33 to kWideMaxK: the MFMA scan keeps 32 per lane list with no shared bound (each list holds
// the 32 best of its own rows), and the merge takes the best sel_n = k + max(16, k / 2) keys over
// all lists, re-scores them exactly and sorts them. A list all 32 of whose entries were taken may
// have held more of the answer: that query runs on the exact kernel instead (fallback list).
constexpr uint32_t kWideMaxK = 256;
constexpr uint32_t kWideMaxSel = 512;

__global__ void __launch_bounds__(256) flat_merge_wide_kernel(MergeArgs m, uint32_t sel_n) {
  constexpr int KL = 32;
  __shared__ uint64_t s_sel[4][kWideMaxSel];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t q = blockIdx.x * 4 + wave;
  if (q >= m.nq) return;  // whole wave; this kernel has no block barriers
  uint64_t* sel = s_sel[wave];
  const float* pd = m.part_d + static_cast<size_t>(q) * m.nlists * KL;
  const uint32_t* pr = m.part_r + static_cast<size_t>(q) * m.nlists * KL;
  uint32_t ptr[kMaxListsPerLane];
  uint64_t head[kMaxListsPerLane];
#pragma unroll
  for (int u = 0; u < kMaxListsPerLane; ++u) {
    const uint32_t li = lane + 64 * u;
    ptr[u] = 0;
    head[u] = li < m.nlists ? make_key(pd[li * KL], pr[li * KL]) : ~0ull;
  }
  uint32_t count = 0;
  bool spent = false;  // one of this lane's lists gave all of its KL entries
  for (uint32_t x = 0; x < sel_n; ++x) {
    uint64_t mine = head[0];
    int arg = 0;
#pragma unroll
    for (int u = 1; u < kMaxListsPerLane; ++u) {
      if (head[u] < mine) {
        mine = head[u];
        arg = u;
      }
    }
    const uint64_t best = wave_min_u64(mine);
    if (static_cast<uint32_t>(best) == QVH_EMPTY_ROW) break;  // only empty slots remain
    if (lane == 0) sel[x] = best;
    ++count;
    if (mine == best) {
#pragma unroll
      for (int u = 0; u < kMaxListsPerLane; ++u) {
        if (u == arg) {
          const uint32_t li = lane + 64 * u;
          const uint32_t p = ++ptr[u];
          if (p < KL) {
            head[u] = make_key(pd[li * KL + p], pr[li * KL + p]);
          } else {
            head[u] = ~0ull;
            spent = spent || x + 1 < sel_n;  // taken before the selection ended
          }
        }
      }
    }
  }
  if (__ballot(spent) != 0) {
    if (lane == 0) m.fallback[atomicAdd(m.nfallback, 1u)] = q;
    return;
  }
  __builtin_amdgcn_wave_barrier();
  // Re-score the selected candidates exactly and rank them by (distance, row).
  uint64_t x8[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t e = static_cast<uint32_t>(i * 64 + lane);
    x8[i] = ~0ull;
    if (e < count) {
      const uint32_t pos = static_cast<uint32_t>(sel[e]);
      const uint32_t row = m.idx ? m.idx[pos] : pos;
      const float d = exact_flat_distance(m.Q + static_cast<size_t>(q) * m.dp, m.X + static_cast<size_t>(row) * m.dp,
                                          m.dim, m.l2 != 0);
      x8[i] = make_key(d, row);
    }
  }
  wave_sort<8>(x8);
  // Certificate: the k-th smallest exact distance (element k - 1) against the sel_n-th selected
  // GEMM-form distance.
  const uint32_t ek_at = m.k - 1;
  uint64_t ek_key = x8[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) ek_key = ek_at / 64 == static_cast<uint32_t>(i) ? x8[i] : ek_key;
  ek_key = __shfl(ek_key, static_cast<int>(ek_at % 64), 64);
  const float e_k = ordered_to_float(static_cast<uint32_t>(ek_key >> 32));
  const float g_last = count == sel_n ? ordered_to_float(static_cast<uint32_t>(sel[sel_n - 1] >> 32)) : 0.0f;
  if (!selection_certified(count, sel_n, g_last, e_k, m.delta[q])) {
    if (lane == 0) m.fallback[atomicAdd(m.nfallback, 1u)] = q;
    return;
  }
  uint32_t* orow = m.out_rows + static_cast<size_t>(q) * m.k;
  float* odist = m.out_dist + static_cast<size_t>(q) * m.k;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t e = static_cast<uint32_t>(i * 64 + lane);
    if (e < m.k) {
      const bool full = e < count;
      orow[e] = full ? static_cast<uint32_t>(x8[i]) : QVH_EMPTY_ROW;
      odist[e] = full ? ordered_to_float(static_cast<uint32_t>(x8[i] >> 32)) : __builtin_huge_valf();
    }
  }
}

// ---- ingest / prep kernels ------------------------------------------------------------------

/// dst[r][c] = c < dim ? src[r][c] : 0 for r < n, c < dp.
__global__ void pack_rows_kernel(const float* __restrict__ src, float* __restrict__ dst, uint64_t n,
                                 uint32_t dim, uint32_t dp) {
  const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= n * dp) return;
  const uint64_t r = idx / dp;
  const uint32_t c = static_cast<uint32_t>(idx % dp);
  dst[idx] = c < dim ? src[r * dim + c] : 0.0f;
}

/// True when v is an integer of magnitude at most 2^24 (exactly representable, and so are its
/// products and sums while they stay below 2^24).
__device__ __forceinline__ bool small_integer(float v) { return v == rintf(v) && fabsf(v) <= 16777216.0f; }

/// Squared norm of one padded row (fused chain over dp / 4 float4 chunks) and whether all of its
/// values are small integers.
__device__ __forceinline__ float padded_norm(const float* row, uint32_t dp, bool& integral) {
  const f32x4* p = reinterpret_cast<const f32x4*>(row);
  float s = 0.0f;
  bool ok = true;
  for (uint32_t c = 0; c < dp / 4; ++c) {
    const f32x4 v = p[c];
    ok = ok && small_integer(v[0]) && small_integer(v[1]) && small_integer(v[2]) && small_integer(v[3]);
    s = fmaf(v[0], v[0], s);
    s = fmaf(v[1], v[1], s);
    s = fmaf(v[2], v[2], s);
    s = fmaf(v[3], v[3], s);
  }
  integral = ok;
  return s;
}

/// out[r] = sum of squares of row r (any order: only the GEMM-form screening uses it). With
/// `meta`, also folds the rows into the store's bound data: meta[0] = largest squared norm (as
/// float bits; non-negative floats order like their bits), meta[1] != 0 once a row holds a value
/// that is not a small integer. One atomic per wave.
__global__ void row_norms_kernel(const float* __restrict__ rows, float* __restrict__ out, uint64_t n,
                                 uint32_t dp, uint32_t* __restrict__ meta) {
  const uint64_t r = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  bool integral = true;
  float s = 0.0f;
  if (r < n) {
    s = padded_norm(rows + r * dp, dp, integral);
    out[r] = s;
  }
  if (meta == nullptr) return;
  uint32_t top = __float_as_uint(s == s ? s : __builtin_huge_valf());
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) top = max(top, static_cast<uint32_t>(__shfl_xor(top, off, 64)));
  const bool all_integral = __ballot(!integral) == 0;
  if ((threadIdx.x & 63) == 0) {
    atomicMax(&meta[0], top);
    if (!all_integral) atomicOr(&meta[1], 1u);
  }
}

/// The queries in the scans' layout, one wave per query: row q of src (dim floats) into qp (dp
/// floats, zero padded); thr_stride words of thr (nullable) per query to +inf and fb[0]
/// (nullable) to zero. With qn, also ||q||^2 into qn (summed in any order: the GEMM form and the
/// bound take any) and the query's bound on |GEMM-form distance - exact distance| over every stored
/// row into delta (the certificate of the MFMA scan's re-score; n = dp rounding steps on any
/// product's path, u = 2^-24, P = ||q||, R = the largest stored ||x||):
///   L2:            |g - e| <= (2n + 4) u (P + R)^2 (1 + O(nu))
///   inner product: |g - e| <= (2n + 2) u (1 + P R) (1 + O(nu))
/// from the standard bound gamma_n = nu / (1 - nu) on a sum of n rounded terms, applied to the
/// GEMM form ||q||^2 + ||x||^2 - 2<q,x> and to the reference's sum of squared differences (or to
/// the two dot products). delta uses the coefficient (4n + 16): a factor of two over the
/// derivation covers the O(nu) terms, the rounding of the computed norms P and R, and a matrix
/// unit whose accumulation rounds faithfully rather than to nearest. delta is 0 when the query
/// and every stored row are small integers and (P + R)^2 <= 2^24: every product, partial sum and
/// difference of either form is then an integer below 2^24, so both forms are exact.
/// *any_delta (nullable) is raised when some query's delta is not 0.
__global__ void __launch_bounds__(256) prep_queries_kernel(const float* __restrict__ src, float* __restrict__ qp,
                                                           uint64_t nq, uint32_t dim, uint32_t dp,
                                                           float* __restrict__ qn, const uint32_t* __restrict__ meta,
                                                           int l2, float* __restrict__ delta,
                                                           uint32_t* __restrict__ any_delta, uint32_t* __restrict__ fb,
                                                           uint32_t* __restrict__ thr, uint32_t thr_stride) {
  const uint64_t q = static_cast<uint64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (q >= nq) return;  // the whole wave
  const uint32_t lane = threadIdx.x & 63u;
  // The search's words for the kernels after this one: the query's shared prune bounds to +inf
  // (ordered bits) and the fallback count to zero.
  if (thr != nullptr && lane < thr_stride) thr[q * thr_stride + lane] = 0xFF800000u;
  if (fb != nullptr && q == 0 && lane == 0) fb[0] = 0u;
  float s = 0.0f;
  bool ok = true;
  for (uint32_t c = lane; c < dp; c += 64) {
    const float v = c < dim ? src[q * dim + c] : 0.0f;
    qp[q * dp + c] = v;
    s = fmaf(v, v, s);
    ok = ok && small_integer(v);
  }
  if (qn == nullptr) return;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  const bool integral = __builtin_amdgcn_ballot_w64(!ok) == 0;
  if (lane != 0) return;
  qn[q] = s;
  const double P = sqrt(static_cast<double>(s));
  const double R = sqrt(static_cast<double>(__uint_as_float(meta[0])));
  const double u = 1.0 / 16777216.0;
  const double coef = (4.0 * dp + 16.0) * u;
  double d;
  if (integral && meta[1] == 0 && (P + R) * (P + R) * (1.0 + 1e-12) <= 16777216.0) {
    d = 0.0;
  } else if (l2) {
    d = coef * (P + R) * (P + R);
  } else {
    d = coef * (1.0 + P * R);
  }
  const float df = static_cast<float>(d);
  delta[q] = static_cast<double>(df) < d ? __uint_as_float(__float_as_uint(df) + 1u) : df;
  if (any_delta != nullptr && d != 0.0) atomicOr(any_delta, 1u);
}

/// Copies the listed rows idx[0..n) of a [rows][4 * c4] store into a contiguous [n][4 * c4] copy,
/// 16 bytes per thread and step (a row's chunks on adjacent lanes), and their squared norms into
/// norms_out when that is set.
__global__ void gather_rows_kernel(const float* __restrict__ X, const float* __restrict__ norms,
                                   const uint32_t* __restrict__ idx, uint64_t n, uint32_t c4, float* __restrict__ out,
                                   float* __restrict__ norms_out) {
  const uint64_t total = n * c4;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint64_t pos = i / c4;
    const uint32_t col = static_cast<uint32_t>(i - pos * c4);
    const uint64_t row = idx[pos];
    reinterpret_cast<f32x4*>(out)[i] = reinterpret_cast<const f32x4*>(X)[row * c4 + col];
    if (norms_out != nullptr && col == 0) norms_out[pos] = norms[row];
  }
}

__global__ void fill_u32_kernel(uint32_t* p, uint64_t n, uint32_t v) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---- general exact search: k above the register lists, or dim above the MFMA query width -----------
//
// One work-group of four waves per query computes every admitted row's distance in the
// reference's arithmetic (so no re-score is needed) and keeps the k best in wave queues cut by
// wave_cut; the four lists are then sorted together.

constexpr int kExactThreads = 256;
constexpr int kExactWaves = kExactThreads / 64;
constexpr uint32_t kExactMaxK = 1024;
// Batches of at most kSplitMaxQueries queries split each query's rows over up to kMaxRowSplits
// work-groups of the exact kernel (at least kMinSplitRows rows each), then merge the sorted lists.
constexpr uint64_t kSplitMaxQueries = 8;
constexpr uint32_t kMaxRowSplits = 1024;
constexpr uint64_t kMinSplitRows = 1024;

struct ExactArgs {
  const float* X;  // [n][dp] rows as stored
  uint32_t dp, dim;
  uint64_t n;
  const float* Q;  // [nq][dp] prepared queries
  uint32_t k;
  int l2;
  const uint64_t* bitmap;
  uint32_t* out_rows;
  float* out_dist;
  const uint32_t* qlist;   // queries to run (block b runs qlist[qskip + b] while qskip + b < *qcount),
  const uint32_t* qcount;  // or null: all. With row splits: list entries 0..nq-1, output slot = entry.
  uint32_t qskip;
  const uint32_t* idx;     // admitted rows, ascending, at positions 0..n-1 (bitmap unused), or null
  // Row splits (nsplit > 1, a multiple of 8; qlist unused): split g scans rows
  // [g * rows_per_split, (g + 1) * rows_per_split) and writes its k best to slot q * nsplit + g of
  // out_rows / out_dist. Work-group b runs on XCD b % 8; it takes query (b / 8) % nq of split
  // ((b / 8) / nq) * 8 + b % 8, so the nq work-groups of one split run together on one XCD and
  // read its rows through the same L2.
  uint32_t nsplit;
  uint32_t nq;
  uint64_t rows_per_split;
};

template <int CAP>
__global__ void __launch_bounds__(kExactThreads) flat_exact_kernel(ExactArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char e_raw[];
  uint64_t* s_queue = reinterpret_cast<uint64_t*>(e_raw);  // [waves][CAP]
  __shared__ uint32_t s_thr;
  __shared__ uint32_t s_wcount[kExactWaves];
  constexpr int QN = CAP / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  uint32_t q = blockIdx.x, split = 0, oslot = 0;
  if (a.nsplit > 1) {
    const uint32_t j = blockIdx.x >> 3;
    q = j % a.nq;
    split = (j / a.nq) * 8 + (blockIdx.x & 7);
    oslot = q;
    if (a.qlist) {
      if (q >= *a.qcount) return;  // block-uniform, before any barrier
      q = a.qlist[q];
    }
  } else if (a.qlist) {
    if (a.qskip + blockIdx.x >= *a.qcount) return;  // block-uniform, before any barrier
    q = a.qlist[a.qskip + blockIdx.x];
    oslot = q;
  } else {
    oslot = q;
  }
  const float* qv = a.Q + static_cast<uint64_t>(q) * a.dp;
  if (tid == 0) s_thr = 0xFFFFFFFFu;
  __syncthreads();
  uint64_t* queue = s_queue + wave * CAP;
  uint32_t cnt = 0;
  uint32_t thr_bits = 0xFFFFFFFFu;
  float thr = __builtin_huge_valf();
  auto cut = [&]() {
    uint32_t t = thr_bits;
    const uint32_t before = cnt;
    cnt = wave_cut<CAP>(queue, cnt, a.k, &t);
    if (before > a.k) {
      if (lane == 0) atomicMin(&s_thr, t);
      if (t < thr_bits) {
        thr_bits = t;
        thr = ordered_to_float(t);
      }
    }
  };
  const uint64_t r_begin = min(a.n, static_cast<uint64_t>(split) * a.rows_per_split);
  const uint64_t r_end = a.nsplit > 1 ? min(a.n, r_begin + a.rows_per_split) : a.n;
  const uint64_t slot = static_cast<uint64_t>(oslot) * max(a.nsplit, 1u) + split;
  for (uint64_t r0 = r_begin; r0 < r_end; r0 += kExactThreads) {
    uint64_t r = r0 + tid;
    bool ok = r < r_end;
    if (ok && a.idx) r = a.idx[r];
    if (ok && a.bitmap && !a.idx) ok = (a.bitmap[r >> 6] >> (r & 63)) & 1ull;
    const float d = ok ? exact_flat_distance(qv, a.X + r * a.dp, a.dim, a.l2 != 0) : 0.0f;
    const bool pass = ok && d <= thr;
    const uint64_t mk = __ballot(pass);
    if (mk != 0) {
      if (pass) queue[cnt + lane_rank(mk)] = make_key(d, static_cast<uint32_t>(r));
      cnt += static_cast<uint32_t>(__popcll(mk));
      if (cnt > static_cast<uint32_t>(CAP - 64)) cut();
    }
    // An atomic load at workgroup scope stays an LDS read; a volatile read of this reference
    // became a flat load whose wait also drained the next step's loads.
    const uint32_t shared_thr = __hip_atomic_load(&s_thr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (shared_thr < thr_bits) {
      thr_bits = shared_thr;
      thr = ordered_to_float(shared_thr);
    }
  }
  cut();
  uint64_t mine[QN];
#pragma unroll
  for (int i = 0; i < QN; ++i) {
    const uint32_t e = i * 64 + lane;
    mine[i] = e < cnt ? queue[e] : ~0ull;
  }
  if (lane == 0) s_wcount[wave] = cnt;
  __syncthreads();
  uint32_t most = 0, merged = 0;
#pragma unroll
  for (int w = 0; w < kExactWaves; ++w) {
    most = max(most, s_wcount[w]);
    merged += s_wcount[w];
  }
  uint32_t ks = 1;
  while (ks < most) ks <<= 1;
#pragma unroll
  for (int i = 0; i < QN; ++i) {
    const uint32_t e = i * 64 + lane;
    if (e < ks) s_queue[wave * ks + e] = mine[i];
  }
  block_sort_keys(s_queue, kExactWaves * ks);
  const uint32_t nout = min(merged, a.k);
  for (uint32_t j = tid; j < a.k; j += kExactThreads) {
    const uint64_t key = j < nout ? s_queue[j] : ~0ull;
    a.out_rows[slot * a.k + j] = j < nout ? static_cast<uint32_t>(key) : QVH_EMPTY_ROW;
    a.out_dist[slot * a.k + j] = j < nout ? ordered_to_float(static_cast<uint32_t>(key >> 32)) : __builtin_huge_valf();
  }
}

// ---------------------------------------------------------------------------------------------
// Few-query exact scan (at most kFewMaxQ queries per launch, 32 <= dim <= kFewMaxDim, k <= 64, or
// k <= kFewMaxK when dim is a multiple of 32).
//
// Eight lanes share a row and load it coalesced: lane l of the eight (u = l & 3, h = l >> 2)
// holds the four accumulators 8u + 4h .. 8u + 4h + 3 of the reference's AVX2 kernel and replays
// their fused chains over the 32-element blocks in order (the 8-element blocks continue the u = 0
// chains in lanes 0 and 4). The horizontal sum then maps onto DPP within the eight lanes:
// quad_perm [1,0,3,2] adds s0 + s1 and s2 + s3, quad_perm [2,3,0,1] gives v = (s0+s1)+(s2+s3) for
// l' = 0..3 (lanes 0-3) and l' = 4..7 (lanes 4-7), row_half_mirror adds the two halves into
// lo[j] = v[j] + v[j+4], and (lo0+lo1)+(lo2+lo3) and the scalar tail finish in each lane. Every
// row is read once for all the launch's queries, whose values stay in registers.

constexpr int kFewThreads = 256;
constexpr int kFewWaves = kFewThreads / 64;
constexpr int kFewRowsPerStep = kFewWaves * 8;
constexpr int kFewCap = 128;  // per (query, wave) queue for k <= 64; 256 for k <= 128
constexpr uint32_t kFewMaxQ = 8;       // queries per launch
// Larger batches take the MFMA scan (1M x 128: 9 queries 357 us in two few-query launches, 295 us on
// the row-split MFMA scan over 256 row splits; 8 queries 274 us in one launch).
constexpr uint32_t kFewMaxBatch = 8;
constexpr uint32_t kFewMaxK = 128;     // dims that are multiples of 32; 64 for the others
constexpr uint32_t kFewMaxDim = 159;  // four 32-element blocks, then up to three 8-blocks and a tail
constexpr uint32_t kFewMaxDp = 160;
constexpr uint32_t kFewMaxSplits = 1024;

struct FewArgs {
  const float* X;  // [n][dp]
  uint32_t dp, dim;
  uint64_t n;
  const float* Q;  // [nq][dp] prepared queries
  uint32_t nq, k;
  const uint64_t* bitmap;
  uint64_t rows_per_split;  // multiple of kFewRowsPerStep
  uint32_t nsplit;
  uint32_t* part_r;  // [nq][nsplit][k]
  float* part_d;
};

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

/// One step's rows for one lane: the four 32-element block pieces and, when the dimension is
/// not a multiple of 32, the 8-element block pieces and the tail.
template <bool TAIL>
struct FewRows {
  float4 x[4];
  float4 xe[TAIL ? 3 : 1];
  float4 t_lo, t_hi;
  uint64_t bits;
};

template <int NQ, bool L2, bool TAIL, int CAP = kFewCap>
__global__ void __launch_bounds__(kFewThreads) flat_few_kernel(FewArgs a) {
  __shared__ uint64_t s_queue[NQ * kFewWaves * CAP];  // [query][wave][CAP]
  __shared__ __attribute__((aligned(16))) float s_q[NQ * kFewMaxDp];
  __shared__ __attribute__((aligned(16))) uint32_t s_thr[NQ < 4 ? 4 : NQ];
  __shared__ uint32_t s_wcount[kFewWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = lane >> 3;  // the wave's row within a step
  const int gl = lane & 7;
  const int u = gl & 3, h = gl >> 2;
  const uint32_t nb = a.dim / 32;              // 32-element blocks (1..4)
  const uint32_t nj = (a.dim - 32 * nb) / 8;   // then 8-element blocks (0..3)
  const uint32_t t0 = 32 * nb + 8 * nj;        // then the scalar tail [t0, dim)
  const uint32_t nt = a.dim - t0;
  const uint32_t nt4 = nt / 4 * 4;             // its first nt4 products are rounded separately

  for (uint32_t i = tid; i < NQ * a.dp; i += kFewThreads) {
    const uint32_t qi = i / a.dp;
    s_q[qi * kFewMaxDp + i % a.dp] = qi < a.nq ? a.Q[static_cast<uint64_t>(qi) * a.dp + i % a.dp] : 0.0f;
  }
  if (tid < (NQ < 4 ? 4 : NQ)) s_thr[tid] = 0xFFFFFFFFu;
  __syncthreads();
  float4 qr[NQ][4];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      qr[qi][b] = b < static_cast<int>(nb) ? *reinterpret_cast<const float4*>(s_q + qi * kFewMaxDp + 32 * b + 8 * u + 4 * h)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
  // In-row offsets of this lane's loads; pieces a dimension does not have re-read block 0 (in
  // bounds, never used), so every load is issued unconditionally and stays in flight.
  uint32_t off_b[4], off_e[3];
#pragma unroll
  for (int b = 0; b < 4; ++b) off_b[b] = b < static_cast<int>(nb) ? 32 * b + 8 * u + 4 * h : 8 * u + 4 * h;
#pragma unroll
  for (int j = 0; j < 3; ++j) off_e[j] = j < static_cast<int>(nj) ? 32 * nb + 8 * j + 4 * h : 4 * h;
  const uint32_t off_t = nt > 0 ? t0 : 0;  // t0 + 8 <= dp when the tail is not empty

  uint32_t cnt[NQ], thr_bits[NQ];
  float thr[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    cnt[qi] = 0;
    thr_bits[qi] = 0xFFFFFFFFu;
    thr[qi] = __builtin_huge_valf();
  }
  auto queue_of = [&](int qi) { return s_queue + (qi * kFewWaves + wave) * CAP; };
  auto cut = [&](int qi) {
    uint32_t t = thr_bits[qi];
    const uint32_t before = cnt[qi];
    cnt[qi] = wave_cut<CAP>(queue_of(qi), cnt[qi], a.k, &t);
    if (before > a.k) {
      if (lane == 0) atomicMin(&s_thr[qi], t);
      if (t < thr_bits[qi]) {
        thr_bits[qi] = t;
        thr[qi] = ordered_to_float(t);
      }
    }
  };

  const uint32_t split = blockIdx.x;
  const uint64_t r_begin = min(a.n, static_cast<uint64_t>(split) * a.rows_per_split);
  const uint64_t r_end = min(a.n, r_begin + a.rows_per_split);
  auto load = [&](uint64_t r0, FewRows<TAIL>& R) {
    uint64_t r = r0 + wave * 8 + grp;
    r = r < r_end ? r : r_begin;  // past the end: a row in range, masked out later
    // The (conditional) bitmap load goes first, so that waiting for this step's rows never
    // waits for the next step's row loads issued after it.
    R.bits = a.bitmap ? a.bitmap[r >> 6] : ~0ull;
    const float* xr = a.X + r * a.dp;
#pragma unroll
    for (int b = 0; b < 4; ++b) R.x[b] = *reinterpret_cast<const float4*>(xr + off_b[b]);
    if constexpr (TAIL) {
#pragma unroll
      for (int j = 0; j < 3; ++j) R.xe[j] = *reinterpret_cast<const float4*>(xr + off_e[j]);
      R.t_lo = *reinterpret_cast<const float4*>(xr + off_t);
      R.t_hi = *reinterpret_cast<const float4*>(xr + off_t + 4);
    }
  };
  FewRows<TAIL> cur;
  if (r_begin < r_end) load(r_begin, cur);
  for (uint64_t r0 = r_begin; r0 < r_end; r0 += kFewRowsPerStep) {
    FewRows<TAIL> nxt;
    load(r0 + kFewRowsPerStep, nxt);  // the next step's rows are in flight while this one computes
    const uint64_t r = r0 + wave * 8 + grp;
    const bool ok = r < r_end && ((cur.bits >> (r & 63)) & 1ull);
    uint32_t shared_thr[NQ];
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) shared_thr[qi] = __hip_atomic_load(&s_thr[qi], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      if (shared_thr[qi] < thr_bits[qi]) {
        thr_bits[qi] = shared_thr[qi];
        thr[qi] = ordered_to_float(shared_thr[qi]);
      }
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
      auto step = [&](const float4& qv, const float4& xv) {
        if constexpr (L2) {
          const float d0 = qv.x - xv.x, d1 = qv.y - xv.y, d2 = qv.z - xv.z, d3 = qv.w - xv.w;
          s0 = fmaf(d0, d0, s0);
          s1 = fmaf(d1, d1, s1);
          s2 = fmaf(d2, d2, s2);
          s3 = fmaf(d3, d3, s3);
        } else {
          s0 = fmaf(qv.x, xv.x, s0);
          s1 = fmaf(qv.y, xv.y, s1);
          s2 = fmaf(qv.z, xv.z, s2);
          s3 = fmaf(qv.w, xv.w, s3);
        }
      };
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (b < static_cast<int>(nb)) step(qr[qi][b], cur.x[b]);
      }
      if constexpr (TAIL) {
        if (u == 0) {
#pragma unroll
          for (int j = 0; j < 3; ++j) {
            if (j < static_cast<int>(nj)) {
              step(*reinterpret_cast<const float4*>(s_q + qi * kFewMaxDp + 32 * nb + 8 * j + 4 * h), cur.xe[j]);
            }
          }
        }
      }
      // horizontal sum, all eight lanes active
      s0 = s0 + dpp_f<0xB1>(s0);
      s1 = s1 + dpp_f<0xB1>(s1);
      s2 = s2 + dpp_f<0xB1>(s2);
      s3 = s3 + dpp_f<0xB1>(s3);
      s0 = s0 + dpp_f<0x4E>(s0);
      s1 = s1 + dpp_f<0x4E>(s1);
      s2 = s2 + dpp_f<0x4E>(s2);
      s3 = s3 + dpp_f<0x4E>(s3);
      s0 = s0 + dpp_f<0x141>(s0);
      s1 = s1 + dpp_f<0x141>(s1);
      s2 = s2 + dpp_f<0x141>(s2);
      s3 = s3 + dpp_f<0x141>(s3);
      float sum = (s0 + s1) + (s2 + s3);
      if constexpr (TAIL) {
        const float xt[8] = {cur.t_lo.x, cur.t_lo.y, cur.t_lo.z, cur.t_lo.w,
                             cur.t_hi.x, cur.t_hi.y, cur.t_hi.z, cur.t_hi.w};
        const float* qt = s_q + qi * kFewMaxDp + t0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (static_cast<uint32_t>(i) < nt) {
            if constexpr (L2) {
              const float d = qt[i] - xt[i];
              sum = static_cast<uint32_t>(i) < nt4 ? sum + d * d : fmaf(d, d, sum);
            } else {
              sum = static_cast<uint32_t>(i) < nt4 ? sum + qt[i] * xt[i] : fmaf(qt[i], xt[i], sum);
            }
          }
        }
      }
      float dist = L2 ? sum : 1.0f - sum;
      dist = dist == dist ? dist : __builtin_huge_valf();
      const bool pass = ok && gl == 0 && static_cast<uint32_t>(qi) < a.nq && dist <= thr[qi];
      const uint64_t mk = __ballot(pass);
      if (mk != 0) {
        if (pass) queue_of(qi)[cnt[qi] + lane_rank(mk)] = make_key(dist, static_cast<uint32_t>(r));
        cnt[qi] += static_cast<uint32_t>(__popcll(mk));
        if (cnt[qi] > static_cast<uint32_t>(CAP - 8)) cut(qi);
      }
    }
    cur = nxt;
  }
  // Per query: the four wave lists (at most CAP / 2 keys each after the cut) sorted together.
  constexpr int MK = CAP / 128;  // keys per lane
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    cut(qi);
    uint64_t mine[MK];
#pragma unroll
    for (int i = 0; i < MK; ++i) {
      const uint32_t e = i * 64 + lane;
      mine[i] = e < cnt[qi] ? queue_of(qi)[e] : ~0ull;
    }
    if (lane == 0) s_wcount[wave] = cnt[qi];
    __syncthreads();
    uint32_t most = 0, merged = 0;
#pragma unroll
    for (int w = 0; w < kFewWaves; ++w) {
      most = max(most, s_wcount[w]);
      merged += s_wcount[w];
    }
    uint32_t ks = 1;
    while (ks < most) ks <<= 1;
    uint64_t* base = s_queue + qi * kFewWaves * CAP;
#pragma unroll
    for (int i = 0; i < MK; ++i) {
      const uint32_t e = i * 64 + lane;
      if (e < ks) base[wave * ks + e] = mine[i];
    }
    block_sort_keys(base, kFewWaves * ks);
    if (static_cast<uint32_t>(qi) < a.nq) {
      const uint32_t nout = min(merged, a.k);
      const uint64_t slot = static_cast<uint64_t>(qi) * a.nsplit + split;
      for (uint32_t j = tid; j < a.k; j += kFewThreads) {
        const uint64_t key = j < nout ? base[j] : ~0ull;
        a.part_r[slot * a.k + j] = j < nout ? static_cast<uint32_t>(key) : QVH_EMPTY_ROW;
        a.part_d[slot * a.k + j] = j < nout ? ordered_to_float(static_cast<uint32_t>(key >> 32)) : __builtin_huge_valf();
      }
    }
    __syncthreads();  // s_wcount is reused by the next query
  }
}

/// The k best of query q's nsplit sorted partial lists of k exact keys each (rows past a list's
/// count are QVH_EMPTY_ROW), by one wave: each step takes the wave minimum of the lanes' list heads
/// (lists lane, lane + 64, ... per lane, up to 64 * LPL lists). A list's next key is loaded one pop
/// ahead, so a step waits on memory only when the same list wins twice in a row.
template <int LPL>
__device__ void merge_sorted_lists(const uint32_t* __restrict__ part_r, const float* __restrict__ part_d, uint32_t q,
                                   uint32_t nsplit, uint32_t k, uint32_t* __restrict__ out_rows,
                                   float* __restrict__ out_dist) {
  const int lane = threadIdx.x & 63;
  const uint32_t* pr = part_r + static_cast<uint64_t>(q) * nsplit * k;
  const float* pd = part_d + static_cast<uint64_t>(q) * nsplit * k;
  auto key_at = [&](uint32_t li, uint32_t p) {
    const uint64_t o = static_cast<uint64_t>(li) * k + p;
    return make_key(pd[o], pr[o]);
  };
  uint32_t ptr[LPL];
  uint64_t head[LPL], next[LPL];
#pragma unroll
  for (int u = 0; u < LPL; ++u) {
    const uint32_t li = lane + 64 * u;
    ptr[u] = 0;
    head[u] = li < nsplit ? key_at(li, 0) : ~0ull;
    next[u] = li < nsplit && k > 1 ? key_at(li, 1) : ~0ull;
  }
  uint32_t* orow = out_rows + static_cast<uint64_t>(q) * k;
  float* odist = out_dist + static_cast<uint64_t>(q) * k;
  for (uint32_t x = 0; x < k; ++x) {
    uint64_t mine = head[0];
    int arg = 0;
#pragma unroll
    for (int u = 1; u < LPL; ++u) {
      if (head[u] < mine) {
        mine = head[u];
        arg = u;
      }
    }
    const uint64_t best = wave_min_u64(mine);
    const bool empty = static_cast<uint32_t>(best) == QVH_EMPTY_ROW;
    if (empty) {
      for (uint32_t y = x + lane; y < k; y += 64) {
        orow[y] = QVH_EMPTY_ROW;
        odist[y] = __builtin_huge_valf();
      }
      return;
    }
    if (lane == 0) {
      orow[x] = static_cast<uint32_t>(best);
      odist[x] = ordered_to_float(static_cast<uint32_t>(best >> 32));
    }
    if (mine == best) {  // one lane: keys are distinct (rows differ)
#pragma unroll
      for (int u = 0; u < LPL; ++u) {
        if (u == arg) {
          const uint32_t p = ++ptr[u];
          head[u] = next[u];
          next[u] = p + 1 < k ? key_at(lane + 64 * u, p + 1) : ~0ull;
        }
      }
    }
  }
}

/// The k best of a query's nsplit <= 1024 sorted partial lists of k <= 256 exact keys each, one
/// 1024-thread work-group per query: T0 is the k-th smallest list head; every key of the k best
/// is <= T0. The heads are distinct keys (a row lives in one split), so at most k lists have a
/// head <= T0, and only they hold such keys: at most k * k real keys are gathered and sorted. With
/// fewer lists than k, T0 is the padding key and every real key is gathered, nsplit * k < k * k of
/// them. So for k <= 64 the kSelectMergeCap = 4096 buffer always suffices; above, a query that
/// gathers more is flagged (overflow[q] = 1, else 0) for the sequential merge of the same lists,
/// which gives the same k keys. With qlist: work-group b merges slot b for query qlist[b] while
/// b < *qcount.
constexpr uint32_t kSelectMergeMaxK = 256;
constexpr uint32_t kSelectMergeLists = 1024;
constexpr uint32_t kSelectMergeCap = 4096;
constexpr uint32_t kSelectMergeFastK = 11;  // k * k <= 128: the gathered keys fit one wave's sort

__global__ void __launch_bounds__(1024) flat_merge_select_kernel(const uint32_t* __restrict__ part_r,
                                                                 const float* __restrict__ part_d,
                                                                 uint32_t nsplit, uint32_t k,
                                                                 uint32_t* __restrict__ out_rows,
                                                                 float* __restrict__ out_dist,
                                                                 uint32_t* __restrict__ overflow,
                                                                 const uint32_t* __restrict__ qlist = nullptr,
                                                                 const uint32_t* __restrict__ qcount = nullptr) {
  __shared__ uint64_t s_heads[kSelectMergeLists];
  __shared__ uint64_t s_cand[kSelectMergeCap];
  __shared__ uint32_t s_count;
  const uint32_t tid = threadIdx.x;
  const uint32_t q = blockIdx.x;
  if (qlist && q >= *qcount) return;  // block-uniform, before any barrier
  const uint64_t oq = qlist ? qlist[q] : q;
  const uint32_t* pr = part_r + static_cast<uint64_t>(q) * nsplit * k;
  const float* pd = part_d + static_cast<uint64_t>(q) * nsplit * k;
  const uint64_t o = static_cast<uint64_t>(tid) * k;
  const uint64_t head = tid < nsplit ? make_key(pd[o], pr[o]) : ~0ull;
  if (tid == 0) s_count = 0;
  uint64_t t0;
  const bool small_k = k <= kSelectMergeFastK;  // block-uniform
  if (small_k) {
    // Each wave sorts its 64 heads in registers; wave 0 then walks the 16 sorted runs, taking the
    // smallest remaining head k times (lane i < 16 follows run i), instead of a 1024-key block
    // bitonic sort (55 barrier steps).
    __shared__ uint64_t s_t0;
    uint64_t h[1] = {head};
    wave_sort<1>(h);
    s_heads[tid] = h[0];
    __syncthreads();
    if (tid < 64) {
      const uint32_t lane = tid;
      uint32_t at = 0;
      uint64_t cur = lane < 16 ? s_heads[lane * 64] : ~0ull;
      uint64_t m = ~0ull;
      for (uint32_t step = 0; step < k; ++step) {
        m = wave_min_u64(cur);
        if (lane < 16 && cur == m && m != ~0ull) {
          ++at;
          cur = at < 64 ? s_heads[lane * 64 + at] : ~0ull;
        }
      }
      if (lane == 0) s_t0 = m;
    }
    __syncthreads();
    t0 = s_t0;
  } else {
    s_heads[tid] = head;
    block_sort_keys(s_heads, kSelectMergeLists);
    t0 = s_heads[k - 1];
  }
  if (tid < nsplit) {
    // this list's keys <= t0, eight at a time
    for (uint32_t p0 = 0; p0 < k; p0 += 8) {
      uint64_t key[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) key[i] = p0 + i < k ? make_key(pd[o + p0 + i], pr[o + p0 + i]) : ~0ull;
      bool more = true;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool take = more && static_cast<uint32_t>(key[i]) != QVH_EMPTY_ROW && key[i] <= t0;
        if (take) {
          const uint32_t at = atomicAdd(&s_count, 1u);
          if (at < kSelectMergeCap) s_cand[at] = key[i];
        }
        more = take;
      }
      if (!more) break;
    }
  }
  __syncthreads();
  const uint32_t c = s_count;
  if (overflow && tid == 0) overflow[q] = c > kSelectMergeCap ? 1u : 0u;
  if (c > kSelectMergeCap) return;  // block-uniform
  if (small_k) {
    // At most k * k <= 121 keys: wave 0 sorts them in registers and writes the k best.
    if (tid < 64) {
      uint64_t x[2] = {tid < c ? s_cand[tid] : ~0ull, tid + 64 < c ? s_cand[tid + 64] : ~0ull};
      wave_sort<2>(x);  // element e = i * 64 + lane in x[i]
      if (tid < k) {
        const bool real = tid < c;
        out_rows[oq * k + tid] = real ? static_cast<uint32_t>(x[0]) : QVH_EMPTY_ROW;
        out_dist[oq * k + tid] = real ? ordered_to_float(static_cast<uint32_t>(x[0] >> 32)) : __builtin_huge_valf();
      }
    }
    return;
  }
  uint32_t n2 = 1;
  while (n2 < c) n2 <<= 1;
  for (uint32_t i = c + tid; i < n2; i += 1024) s_cand[i] = ~0ull;
  block_sort_keys(s_cand, n2);
  for (uint32_t j = tid; j < k; j += 1024) {
    const bool real = j < c;
    out_rows[oq * k + j] = real ? static_cast<uint32_t>(s_cand[j]) : QVH_EMPTY_ROW;
    out_dist[oq * k + j] = real ? ordered_to_float(static_cast<uint32_t>(s_cand[j] >> 32)) : __builtin_huge_valf();
  }
}

/// One wave per query of merge_sorted_lists (only the queries flagged in `only`, when given).
template <int LPL>
__global__ void __launch_bounds__(256) flat_merge_sorted_kernel(const uint32_t* __restrict__ part_r,
                                                                const float* __restrict__ part_d, uint32_t nq,
                                                                uint32_t nsplit, uint32_t k,
                                                                uint32_t* __restrict__ out_rows,
                                                                float* __restrict__ out_dist,
                                                                const uint32_t* __restrict__ only) {
  const uint32_t q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= nq || (only && only[q] == 0)) return;  // whole wave; no block barriers
  merge_sorted_lists<LPL>(part_r, part_d, q, nsplit, k, out_rows, out_dist);
}

/// The k best of each query's nsplit sorted lists [nq][nsplit][k] into [nq][k]. `flags` ([nq]
/// words) is needed for 64 < k <= kSelectMergeMaxK, where a query's selection can overflow.
void launch_sorted_merge(const uint32_t* part_r, const float* part_d, uint64_t nq, uint32_t nsplit, uint32_t k,
                         uint32_t* d_rows, float* d_dist, uint32_t* flags, hipStream_t s) {
  QVH_REQUIRE(nsplit <= 64 * 16, "flat search: too many partial lists to merge");
  const uint32_t* only = nullptr;
  if (k <= kSelectMergeMaxK) {
    uint32_t* overflow = k > 64 ? flags : nullptr;
    hipLaunchKernelGGL(flat_merge_select_kernel, dim3(static_cast<unsigned>(nq)), dim3(1024), 0, s, part_r, part_d,
                       nsplit, k, d_rows, d_dist, overflow);
    QVH_HIP(hipGetLastError());
    if (!overflow) return;
    only = overflow;  // the sequential merge takes the overflowed queries
  }
  const dim3 grid(static_cast<unsigned>(ceil_div(nq, 4))), block(256);
  const uint32_t q32 = static_cast<uint32_t>(nq);
  if (nsplit <= 64) {
    hipLaunchKernelGGL(flat_merge_sorted_kernel<1>, grid, block, 0, s, part_r, part_d, q32, nsplit, k, d_rows, d_dist, only);
  } else if (nsplit <= 128) {
    hipLaunchKernelGGL(flat_merge_sorted_kernel<2>, grid, block, 0, s, part_r, part_d, q32, nsplit, k, d_rows, d_dist, only);
  } else if (nsplit <= 256) {
    hipLaunchKernelGGL(flat_merge_sorted_kernel<4>, grid, block, 0, s, part_r, part_d, q32, nsplit, k, d_rows, d_dist, only);
  } else if (nsplit <= 512) {
    hipLaunchKernelGGL(flat_merge_sorted_kernel<8>, grid, block, 0, s, part_r, part_d, q32, nsplit, k, d_rows, d_dist, only);
  } else {
    hipLaunchKernelGGL(flat_merge_sorted_kernel<16>, grid, block, 0, s, part_r, part_d, q32, nsplit, k, d_rows, d_dist, only);
  }
  QVH_HIP(hipGetLastError());
}

void launch_exact(const ExactArgs& a, uint64_t nq, hipStream_t s) {
  const uint32_t cap = a.k <= 64 ? 128 : a.k <= 128 ? 256 : a.k <= 256 ? 512 : a.k <= 512 ? 1024 : 2048;
  const size_t lds = static_cast<size_t>(kExactWaves) * cap * sizeof(uint64_t);
  auto go = [&](auto kernel) {
    if (lds > 64 * 1024) {
      QVH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(lds)));
    }
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(nq * std::max(1u, a.nsplit))), dim3(kExactThreads), lds, s, a);
  };
  switch (cap) {
    case 128: go(flat_exact_kernel<128>); break;
    case 256: go(flat_exact_kernel<256>); break;
    case 512: go(flat_exact_kernel<512>); break;
    case 1024: go(flat_exact_kernel<1024>); break;
    default: go(flat_exact_kernel<2048>); break;
  }
  QVH_HIP(hipGetLastError());
}

// ---- k above kExactMaxK: score every admitted row, sort, keep k ------------------------------
//
// FlatIndex::search_batch for any k (src/flat_index.cc:84-107): every admitted row of a query is
// scored in the reference's order, its (distance, row) keys sorted by a segmented radix sort and
// the first k kept; rows not admitted get the largest key and come out as empty slots.
constexpr uint64_t kSortMaxKeys = uint64_t{1} << 26;  // keys per pass (two 512 MiB key buffers)

size_t sorted_scratch_bytes(uint64_t keys, uint32_t segments) {
  size_t bytes = 0;
  QVH_HIP(rocprim::segmented_radix_sort_keys(nullptr, bytes, static_cast<const uint64_t*>(nullptr),
                                             static_cast<uint64_t*>(nullptr), static_cast<unsigned int>(keys),
                                             segments, static_cast<const uint32_t*>(nullptr),
                                             static_cast<const uint32_t*>(nullptr)));
  return std::max<size_t>(bytes, 1);
}

/// keys[y][pos] for query q0 + y and position pos < n (rows, or listed rows idx[pos]).
__global__ void sort_keys_kernel(ExactArgs a, uint32_t q0, uint64_t* __restrict__ keys) {
  const uint64_t pos = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (pos >= a.n) return;
  const uint32_t y = blockIdx.y;
  uint64_t row = pos;
  bool ok = true;
  if (a.idx) {
    row = a.idx[pos];
  } else if (a.bitmap) {
    ok = (a.bitmap[row >> 6] >> (row & 63)) & 1ull;
  }
  uint64_t key = ~0ull;
  if (ok) {
    const float d = exact_flat_distance(a.Q + static_cast<uint64_t>(q0 + y) * a.dp, a.X + row * a.dp, a.dim, a.l2 != 0);
    key = make_key(d, static_cast<uint32_t>(pos));
  }
  keys[static_cast<uint64_t>(y) * a.n + pos] = key;
}

__global__ void sort_offsets_kernel(uint32_t* off, uint32_t segments, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= segments) off[i] = i * n;
}

/// The first k sorted keys of query q0 + y as rows and distances (empty slots past the admitted).
__global__ void sort_take_kernel(const uint64_t* __restrict__ keys, uint64_t n, uint32_t k, uint32_t q0,
                                 const uint32_t* __restrict__ idx, uint32_t* __restrict__ out_rows,
                                 float* __restrict__ out_dist) {
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= k) return;
  const uint32_t y = blockIdx.y;
  const uint64_t key = j < n ? keys[static_cast<uint64_t>(y) * n + j] : ~0ull;
  const uint64_t o = static_cast<uint64_t>(q0 + y) * k + j;
  if (key == ~0ull) {
    out_rows[o] = QVH_EMPTY_ROW;
    out_dist[o] = __builtin_huge_valf();
    return;
  }
  const uint32_t pos = static_cast<uint32_t>(key);
  out_rows[o] = idx ? idx[pos] : pos;
  out_dist[o] = ordered_to_float(static_cast<uint32_t>(key >> 32));
}

/// Workspace of run_sorted: keys [chunk][n] twice, chunk + 1 offsets, the sort's scratch.
struct SortBuffers {
  uint64_t chunk;
  uint64_t* skin;
  uint64_t* skout;
  uint32_t* soff;
  void* stmp;
  size_t stmp_bytes;
};

void run_sorted(const SortBuffers& b, ExactArgs e, uint64_t nq, uint32_t k, hipStream_t s) {
  const uint64_t n = e.n;
  for (uint64_t q0 = 0; q0 < nq; q0 += b.chunk) {
    const uint32_t nc = static_cast<uint32_t>(std::min<uint64_t>(b.chunk, nq - q0));
    if (n > 0) {
      hipLaunchKernelGGL(sort_keys_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256)), nc), dim3(256), 0, s, e,
                         static_cast<uint32_t>(q0), b.skin);
      hipLaunchKernelGGL(sort_offsets_kernel, dim3(static_cast<unsigned>(ceil_div(nc + 1, 256))), dim3(256), 0, s,
                         b.soff, nc, static_cast<uint32_t>(n));
      size_t bytes = b.stmp_bytes;
      QVH_HIP(rocprim::segmented_radix_sort_keys(b.stmp, bytes, b.skin, b.skout, static_cast<unsigned int>(nc * n), nc,
                                                 b.soff, b.soff + 1, 0, 64, s));
    }
    hipLaunchKernelGGL(sort_take_kernel, dim3(static_cast<unsigned>(ceil_div(k, 256)), nc), dim3(256), 0, s, b.skout, n,
                       k, static_cast<uint32_t>(q0), e.idx, e.out_rows, e.out_dist);
    QVH_HIP(hipGetLastError());
  }
}

int device_cus(int device) {
  int cus = 256;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  return cus;
}

/// Listed fallback queries that run over row splits, and their split count for n rows: up to 128
/// splits of at least kMinSplitRows rows (a multiple of 8 for the XCD mapping), about four
/// work-groups per CU in all; 0 when the rows are too few to split.
constexpr uint32_t kFallbackSplitQueries = 8;
uint32_t fallback_splits(uint64_t n, int cus) {
  const uint64_t want = std::max<uint64_t>(8, static_cast<uint64_t>(cus) * 4 / kFallbackSplitQueries);
  const uint64_t g = std::min<uint64_t>({want, 128, n / kMinSplitRows}) / 8 * 8;
  return static_cast<uint32_t>(g);
}

/// Row stride in floats. Up to kMaxDp (the register-resident scan): the dimension rounded up to 8,
/// at least 16 (each MFMA lane half takes dp / 2 dims in float4 steps, and a row stride of dp + 4
/// floats is an odd multiple of 4, which keeps the b128 tile reads conflict-free); dim 100 runs 53
/// MFMA steps per tile instead of 57. Wider rows: rounded up to 16 (the chunked scan).
uint32_t padded_dim(uint32_t dim) {
  if (dim <= static_cast<uint32_t>(kMaxDp)) return std::max(16u, (dim + 7u) / 8u * 8u);
  return (dim + 15u) / 16u * 16u;
}

/// Per-lane list length of the MFMA scan for k, or 0 when k needs the wide merge. A margin of
/// max(5, k/2) candidates past k lets the merge's re-score certify the selection when the GEMM-form
/// distances differ from the exact ones in rounding.
int shared_list_length(uint32_t k) {
  const uint32_t need = k + std::max(5u, k / 2);
  return need <= 16 ? 16 : need <= 32 ? 32 : 0;
}

/// List length for a batch whose GEMM-form distances are all exact (every query's delta is 0:
/// small-integer queries against a store of small integers), which needs no margin over k; 0 when
/// none applies. 1M x 128 integer mixture, k = 10: scan 22.30 -> 21.53 ms, merge 82 -> 65 us (12
/// entries: 21.79 ms).
int exact_list_length(uint32_t k) { return k <= 10 ? 10 : 0; }

template <int DP, int KL>
void launch_scan_kl(bool l2, int mode, dim3 grid, const ScanArgs& a, hipStream_t s) {
  if (a.rowsplit) {  // unfiltered batches of at most 128 queries
    if (l2) {
      hipLaunchKernelGGL((flat_scan_kernel<DP, KL, true, 0, true>), grid, dim3(kThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL((flat_scan_kernel<DP, KL, false, 0, true>), grid, dim3(kThreads), 0, s, a);
    }
    return;
  }
  if (l2) {
    if (mode == 1) {
      hipLaunchKernelGGL((flat_scan_kernel<DP, KL, true, 1>), grid, dim3(kThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL((flat_scan_kernel<DP, KL, true, 0>), grid, dim3(kThreads), 0, s, a);
    }
  } else {
    if (mode == 1) {
      hipLaunchKernelGGL((flat_scan_kernel<DP, KL, false, 1>), grid, dim3(kThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL((flat_scan_kernel<DP, KL, false, 0>), grid, dim3(kThreads), 0, s, a);
    }
  }
}

template <int DP>
void launch_scan_dp(int kl, bool l2, int mode, dim3 grid, const ScanArgs& a, hipStream_t s) {
  if (kl == 10) {
    launch_scan_kl<DP, 10>(l2, mode, grid, a, s);
  } else if (kl == 16) {
    launch_scan_kl<DP, 16>(l2, mode, grid, a, s);
  } else {
    launch_scan_kl<DP, 32>(l2, mode, grid, a, s);
  }
}

template <int KL>
void launch_scan_chunked_kl(bool l2, int mode, dim3 grid, const ScanArgs& a, hipStream_t s) {
  if (l2) {
    if (mode == 1) {
      hipLaunchKernelGGL((flat_scan_k_kernel<KL, true, 1>), grid, dim3(kThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL((flat_scan_k_kernel<KL, true, 0>), grid, dim3(kThreads), 0, s, a);
    }
  } else {
    if (mode == 1) {
      hipLaunchKernelGGL((flat_scan_k_kernel<KL, false, 1>), grid, dim3(kThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL((flat_scan_k_kernel<KL, false, 0>), grid, dim3(kThreads), 0, s, a);
    }
  }
}

/// The MFMA scan for padded width dp: register-resident queries up to kMaxDp, chunked above.
void launch_scan(uint32_t dp, int kl, dim3 grid, const ScanArgs& a, hipStream_t s) {
  const bool l2 = a.l2 != 0;
  const int filter = a.bitmap ? 1 : 0;
  if (dp > static_cast<uint32_t>(kMaxDp)) {
    if (kl == 10) {
      launch_scan_chunked_kl<10>(l2, filter, grid, a, s);
    } else if (kl == 16) {
      launch_scan_chunked_kl<16>(l2, filter, grid, a, s);
    } else {
      launch_scan_chunked_kl<32>(l2, filter, grid, a, s);
    }
    return;
  }
  switch (dp) {
    case 16: launch_scan_dp<16>(kl, l2, filter, grid, a, s); break;
    case 24: launch_scan_dp<24>(kl, l2, filter, grid, a, s); break;
    case 32: launch_scan_dp<32>(kl, l2, filter, grid, a, s); break;
    case 40: launch_scan_dp<40>(kl, l2, filter, grid, a, s); break;
    case 48: launch_scan_dp<48>(kl, l2, filter, grid, a, s); break;
    case 56: launch_scan_dp<56>(kl, l2, filter, grid, a, s); break;
    case 64: launch_scan_dp<64>(kl, l2, filter, grid, a, s); break;
    case 72: launch_scan_dp<72>(kl, l2, filter, grid, a, s); break;
    case 80: launch_scan_dp<80>(kl, l2, filter, grid, a, s); break;
    case 88: launch_scan_dp<88>(kl, l2, filter, grid, a, s); break;
    case 96: launch_scan_dp<96>(kl, l2, filter, grid, a, s); break;
    case 104: launch_scan_dp<104>(kl, l2, filter, grid, a, s); break;
    case 112: launch_scan_dp<112>(kl, l2, filter, grid, a, s); break;
    case 120: launch_scan_dp<120>(kl, l2, filter, grid, a, s); break;
    case 128: launch_scan_dp<128>(kl, l2, filter, grid, a, s); break;
    default: throw Failure(QVH_EUNSUPPORTED, "flat scan: unsupported padded dimension");
  }
}

template <int DP>
void launch_ring_dp(int kl, bool l2, dim3 grid, const ScanArgs& a, hipStream_t s) {
  auto go = [&](auto klc) {
    constexpr int KL = decltype(klc)::value;
    if (l2) {
      hipLaunchKernelGGL((flat_ring_kernel<DP, KL, true>), grid, dim3(kRingThreads), 0, s, a);
    } else {
      hipLaunchKernelGGL((flat_ring_kernel<DP, KL, false>), grid, dim3(kRingThreads), 0, s, a);
    }
  };
  if (kl == 10) {
    go(std::integral_constant<int, 10>{});
  } else if (kl == 16) {
    go(std::integral_constant<int, 16>{});
  } else {
    go(std::integral_constant<int, 32>{});
  }
}

/// The ring scan for padded width dp (a multiple of 32 up to kMaxDp), one work-group per split.
void launch_ring(uint32_t dp, int kl, dim3 grid, const ScanArgs& a, hipStream_t s) {
  const bool l2 = a.l2 != 0;
  switch (dp) {
    case 32: launch_ring_dp<32>(kl, l2, grid, a, s); break;
    case 64: launch_ring_dp<64>(kl, l2, grid, a, s); break;
    case 96: launch_ring_dp<96>(kl, l2, grid, a, s); break;
    case 128: launch_ring_dp<128>(kl, l2, grid, a, s); break;
    default: throw Failure(QVH_EUNSUPPORTED, "ring scan: padded dimension is not a multiple of 32 up to 128");
  }
}

}  // namespace

struct qvh_flat {
  uint32_t dim = 0, dp = 0;
  int metric = 0;
  int device = 0;
  uint64_t n = 0, cap = 0;
  DeviceBuffer rows, norms;
  // meta[0]: largest stored squared norm (float bits), meta[1]: nonzero once a stored value is not a
  // small integer (row_norms_kernel); the inputs of the re-score certificate's bound.
  DeviceBuffer meta;
  // Host copy of meta after the last append: every stored value a small integer and every stored
  // squared norm at most 2^24, so that integer queries re-score with delta = 0.
  bool integral_rows = true;
  uint32_t h_meta[2] = {0, 0};
  hipStream_t stream = nullptr;
  std::mutex mu;
  // per-call workspace (grown on demand, serialized by mu)
  DeviceBuffer w_stage, w_q, w_qn, w_pd, w_pr, w_rows, w_dist, w_bits, w_thr, w_idx, w_fb, w_mflag, w_delta;
  DeviceBuffer w_skin, w_skout, w_soff, w_stmp;  // k above kExactMaxK: sort keys and scratch
  DeviceBuffer w_cx, w_cn;                        // listed rows gathered for the MFMA scan, their norms
  // optional per-stage timing of the last search: events before prep, scan, merge and after
  bool timing = false;
  bool timed = false;
  hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
  hipEvent_t join = nullptr;  // orders calls on other streams into the handle's stream
  uint64_t last_nsplit = 0;
  bool last_fb = false;               // the last search took the MFMA scan
  uint32_t* last_fb_count = nullptr;  // where its fallback count went (device memory)
};

namespace {

void flat_grow(qvh_flat* f, uint64_t need) {
  if (need <= f->cap) return;
  uint64_t cap = std::max<uint64_t>(need, f->cap ? f->cap * 2 : 1024);
  void* nr = device_alloc(cap * f->dp * sizeof(float));
  void* nn = nullptr;
  try {
    nn = device_alloc(cap * sizeof(float));
  } catch (...) {
    device_free(nr);
    throw;
  }
  if (f->n) {
    QVH_HIP(hipMemcpyAsync(nr, f->rows.ptr, f->n * f->dp * sizeof(float), hipMemcpyDeviceToDevice, f->stream));
    QVH_HIP(hipMemcpyAsync(nn, f->norms.ptr, f->n * sizeof(float), hipMemcpyDeviceToDevice, f->stream));
    QVH_HIP(hipStreamSynchronize(f->stream));
  }
  device_free(f->rows.ptr);
  device_free(f->norms.ptr);
  f->rows.ptr = nr;
  f->rows.bytes = cap * f->dp * sizeof(float);
  f->norms.ptr = nn;
  f->norms.bytes = cap * sizeof(float);
  f->cap = cap;
}

/// One search's path, launch geometry and workspace, decided on the host before anything is
/// launched, so a caller with a fixed workspace can be refused up front.
struct FlatPlan {
  enum Path { kFew, kSplit, kExactOnly, kMfma, kSorted } path = kMfma;
  bool wide = false;
  bool ring = false;  // kMfma: the ring scan (one 32-query group, unfiltered) instead of the MFMA scan
  int kl = 16;
  // List length when every query's distances turn out exact (exact_list_length), or 0: the scan
  // and merge are then launched for both lengths, and the device runs the one that applies.
  int kl_exact = 0;
  uint64_t g = 0, rps = 0;                       // few / split: row splits and rows per split
  uint64_t nsplit = 1, rows_per_split = 0;       // MFMA scan
  uint32_t qblocks = 0;
  uint64_t scan_rows = 0;
  // Bytes of each workspace buffer (0 = unused).
  size_t stage = 0, q = 0, qn = 0, delta = 0, pd = 0, pr = 0, thr = 0, fb = 0, mflag = 0;
  // Listed rows for the MFMA scan: their contiguous copy and (L2) its squared norms.
  size_t cx = 0, cn = 0;
  // k above kExactMaxK: sort_chunk queries per pass; two key buffers, segment offsets, sort scratch.
  uint64_t sort_chunk = 0;
  size_t skeys = 0, soff = 0, stmp = 0;

  static size_t aligned(size_t b) { return (b + 255) / 256 * 256; }
  size_t total() const {
    return aligned(stage) + aligned(q) + aligned(qn) + aligned(delta) + aligned(pd) + aligned(pr) + aligned(thr) +
           aligned(fb) + aligned(mflag) + 2 * aligned(skeys) + aligned(soff) + aligned(stmp) + aligned(cx) +
           aligned(cn);
  }
};

/// The workspace of one search, on the handle's buffers or carved from a caller-fixed region.
struct FlatBuffers {
  float* stage = nullptr;
  float* q = nullptr;
  float* qn = nullptr;
  float* delta = nullptr;
  float* pd = nullptr;
  uint32_t* pr = nullptr;
  uint32_t* thr = nullptr;
  uint32_t* fb = nullptr;
  uint32_t* mflag = nullptr;
  uint64_t* skin = nullptr;
  uint64_t* skout = nullptr;
  uint32_t* soff = nullptr;
  void* stmp = nullptr;
  float* cx = nullptr;
  float* cn = nullptr;
};

/// d_idx (listed admitted rows) is in use when n_idx > 0 or `indexed`.
FlatPlan plan_flat_search(const qvh_flat* f, uint64_t nq, uint32_t k, bool indexed, bool filtered, uint64_t n_idx,
                          int cus) {
  QVH_REQUIRE(nq <= 0xFFFFFFFFull, "flat search: too many queries in one call");
  FlatPlan p;
  if (k > kExactMaxK) {
    // Every admitted row of a query scored exactly and the (distance, row) keys sorted: chunks of
    // queries whose keys fit kSortMaxKeys.
    p.path = FlatPlan::kSorted;
    if (f->metric == QVH_METRIC_COSINE) p.stage = nq * f->dim * sizeof(float);
    p.q = nq * f->dp * sizeof(float);
    const uint64_t n_scan = std::max<uint64_t>(1, indexed ? n_idx : f->n);
    QVH_REQUIRE(n_scan <= kSortMaxKeys, "flat search: too many rows for k above " + std::to_string(kExactMaxK));
    p.sort_chunk = std::max<uint64_t>(1, std::min<uint64_t>(nq, kSortMaxKeys / n_scan));
    p.skeys = p.sort_chunk * n_scan * sizeof(uint64_t);
    p.soff = (p.sort_chunk + 1) * sizeof(uint32_t);
    p.stmp = sorted_scratch_bytes(p.sort_chunk * n_scan, static_cast<uint32_t>(p.sort_chunk));
    return p;
  }
  // At most kFewMaxBatch queries with 32 <= dim <= kFewMaxDim and k <= kFewMaxK: the few-query
  // scan, kFewMaxQ queries per launch;
  // other batches of at most kSplitMaxQueries: the exact kernel over row splits. Otherwise k with a
  // margin in a shared-bound list (shared_list_length): the MFMA scan with per-lane lists of KL = 16
  // or 32 and a shared bound; larger k up to kWideMaxK: the same scan without the shared bound and
  // the wide merge (its rare fallback queries on the exact kernel); larger k or dim: the exact kernel.
  // Rows wider than kMaxDp (up to kMaxChunkedDp) take the chunked form of the MFMA scan.
  // kRingMinQueries to kRingMaxQueries unfiltered queries whose rows are whole 32-dim quarters,
  // with k in the shared-bound lists: the ring scan (its lists go to the same merge as the MFMA
  // scan's); fewer queries too when the rows are too few to split for the few-query kernel.
  const bool ring = !indexed && !filtered && f->n >= 1 && nq <= kRingMaxQueries && shared_list_length(k) != 0 &&
                    f->dp % 32 == 0 && f->dp <= static_cast<uint32_t>(kMaxDp) &&
                    (nq >= kRingMinQueries || f->n < 2 * kMinSplitRows);
  const bool splittable = !indexed && f->n >= 2 * kMinSplitRows;
  const bool few = !ring && splittable && nq <= kFewMaxBatch && k <= (f->dim % 32 == 0 ? kFewMaxK : 64u) &&
                   f->dim >= 32 && f->dim <= kFewMaxDim;
  const bool split = !ring && splittable && !few && nq <= kSplitMaxQueries;
  p.wide = !few && !split && shared_list_length(k) == 0 && k <= kWideMaxK && f->dp <= kMaxChunkedDp &&
           !indexed;
  const bool exact_only = !few && !split && !p.wide && (shared_list_length(k) == 0 || f->dp > kMaxChunkedDp);
  p.path = few ? FlatPlan::kFew : split ? FlatPlan::kSplit : exact_only ? FlatPlan::kExactOnly : FlatPlan::kMfma;
  if (f->metric == QVH_METRIC_COSINE) p.stage = nq * f->dim * sizeof(float);
  p.q = nq * f->dp * sizeof(float);
  if (p.path == FlatPlan::kFew) {
    // A few queries of moderate width: the coalesced few-query kernel reads each row once for
    // each launch of up to kFewMaxQ queries, over enough row splits to give every CU four
    // work-groups; one merge then serves the whole batch.
    uint64_t g = std::min<uint64_t>({static_cast<uint64_t>(kFewMaxSplits), f->n / kMinSplitRows,
                                     static_cast<uint64_t>(cus) * 4});
    p.rps = ceil_div(ceil_div(f->n, g), kFewRowsPerStep) * kFewRowsPerStep;
    p.g = ceil_div(f->n, p.rps);
  } else if (p.path == FlatPlan::kSplit) {
    // A few queries: the MFMA scan's 256-query blocks would run mostly empty. Split each query's
    // rows over enough exact-kernel work-groups to give every CU eight, then merge.
    const uint64_t want = ceil_div(static_cast<uint64_t>(cus) * 8, nq);
    uint64_t g = std::min<uint64_t>({want, kMaxRowSplits, f->n / kMinSplitRows});
    p.rps = ceil_div(ceil_div(f->n, g), kExactThreads) * kExactThreads;
    p.g = ceil_div(ceil_div(f->n, p.rps), 8) * 8;  // the XCD mapping takes whole groups of 8 splits
  }
  if (p.path == FlatPlan::kFew || p.path == FlatPlan::kSplit) {
    const size_t parts = static_cast<size_t>(nq) * p.g * k;
    p.pr = parts * sizeof(uint32_t);
    p.pd = parts * sizeof(float);
    p.mflag = nq * sizeof(uint32_t);
    return p;
  }
  if (p.path == FlatPlan::kExactOnly) return p;
  p.qn = nq * sizeof(float);
  p.delta = nq * sizeof(float);
  p.kl = p.wide ? 32 : shared_list_length(k);
  // The ring scan takes the margin's lists for integer stores too (exact distances certify with any
  // list length): a second, gated launch of its scan and merge would cost more than it saves.
  p.kl_exact = !p.wide && !ring && f->integral_rows ? exact_list_length(k) : 0;
  p.qblocks = static_cast<uint32_t>(ceil_div(nq, kQueriesPerBlock));
  p.scan_rows = indexed ? n_idx : f->n;
  if (ring) {
    // One work-group (160 KB of LDS: one per CU) per split of whole 32-row blocks, as many splits
    // as CUs (at most kRingMaxSplits) while each keeps kRingMinSplitRows rows.
    p.ring = true;
    p.nsplit = std::min<uint64_t>({kRingMaxSplits, static_cast<uint64_t>(std::max(cus, 1)),
                                   std::max<uint64_t>(1, p.scan_rows / kRingMinSplitRows)});
    p.rows_per_split = ceil_div(ceil_div(p.scan_rows, p.nsplit), 32) * 32;
    p.nsplit = ceil_div(p.scan_rows, p.rows_per_split);
  } else {
    const uint64_t tiles = std::max<uint64_t>(1, ceil_div(p.scan_rows, kTileRows));
    // One workgroup per CU at a time: the split count (1 to 7, or a multiple of 8 for the XCD
    // mapping) is the smallest whose workgroups fill whole rounds of the CUs to 97%: longer splits
    // start fewer lists and exchange bounds with fewer others. 1M x 128, scan at k = 10 (the earlier
    // choice, which preferred four rounds, without bound slots above 64 splits -> this one): 512
    // queries 256 -> 128 splits 1.33 -> 1.18 ms, 1,024 queries 256 -> 64 splits 2.46 -> 2.14 ms,
    // 2,048 queries 128 -> 32 splits 4.71 -> 4.12 ms, 8,192 queries 32 -> 8 splits 16.04 -> 15.97 ms;
    // 10,000 queries keep 32 (24 splits: 21.27 ms, 32: 20.22, 40: 22.35). When no count fills 97%
    // of its rounds, the best fill weighted by parallelism (at least four rounds when the rows
    // allow) decides, fewer splits on ties. A split keeps at least four tiles: with fewer
    // rows per split the per-split top-k lists take in most rows (1.18M x 100 cosine with 0.5% of
    // the ids allowed: 32 splits 0.47 ms, 16 splits 0.37 ms).
    {
      const uint64_t cap = std::max<uint64_t>(1, std::min<uint64_t>(tiles / 4, kMaxSplits));
      double best = -1.0;
      bool full = false;
      for (uint64_t c = 1; c <= cap && !full; c = c < 8 ? c + 1 : c + 8) {
        if (c >= 8 && c % 8) continue;
        const uint64_t total = p.qblocks * c;
        const uint64_t rounds = ceil_div(total, static_cast<uint64_t>(cus));
        const double fill = static_cast<double>(total) / static_cast<double>(rounds * cus);
        if (fill >= 0.97) {
          p.nsplit = c;
          full = true;
        }
      }
      for (uint64_t c = 1; c <= cap && !full; c = c < 8 ? c + 1 : c + 8) {
        if (c >= 8 && c % 8) continue;
        const uint64_t total = p.qblocks * c;
        const uint64_t rounds = ceil_div(total, static_cast<uint64_t>(cus));
        const double fill = static_cast<double>(total) / static_cast<double>(rounds * cus);
        const double par = std::min(1.0, static_cast<double>(total) / (4.0 * cus));
        const double score = fill * par;
        if (score > best + 1e-9) {
          best = score;
          p.nsplit = c;
        }
      }
    }
    p.rows_per_split = ceil_div(tiles, p.nsplit) * kTileRows;
  }
  const size_t parts = static_cast<size_t>(nq) * 2 * p.nsplit * p.kl;
  p.pd = parts * sizeof(float);
  p.pr = parts * sizeof(uint32_t);
  p.thr = nq * (p.ring ? kRingBoundStride : kScanBoundStride) * sizeof(uint32_t);
  p.fb = (nq + 2) * sizeof(uint32_t);  // count, listed queries, then the launch gate word
  // Listed rows are gathered once into a contiguous copy: the scan reads every row once per query
  // block, and through the list each of those reads would be a scattered gather (1.18M x 100
  // cosine, 10% listed, 10,000 queries: 2.97 ms through the list, 2.86 ms on the copy).
  if (indexed && n_idx > 0) {
    QVH_REQUIRE(n_idx * f->dp * sizeof(float) <= kCompactMaxBytes, "flat search: too many listed rows");
    p.cx = n_idx * f->dp * sizeof(float);
    p.cn = f->metric == QVH_METRIC_L2 ? n_idx * sizeof(float) : 0;
  }
  return p;
}

/// The plan's workspace on the handle's own buffers (grown on demand).
FlatBuffers handle_buffers(qvh_flat* f, const FlatPlan& p) {
  FlatBuffers b;
  auto take = [](DeviceBuffer& buf, size_t bytes) { return bytes ? buf.reserve(bytes) : nullptr; };
  b.stage = static_cast<float*>(take(f->w_stage, p.stage));
  b.q = static_cast<float*>(take(f->w_q, p.q));
  b.qn = static_cast<float*>(take(f->w_qn, p.qn));
  b.delta = static_cast<float*>(take(f->w_delta, p.delta));
  b.pd = static_cast<float*>(take(f->w_pd, p.pd));
  b.pr = static_cast<uint32_t*>(take(f->w_pr, p.pr));
  b.thr = static_cast<uint32_t*>(take(f->w_thr, p.thr));
  b.fb = static_cast<uint32_t*>(take(f->w_fb, p.fb));
  b.mflag = static_cast<uint32_t*>(take(f->w_mflag, p.mflag));
  b.skin = static_cast<uint64_t*>(take(f->w_skin, p.skeys));
  b.skout = static_cast<uint64_t*>(take(f->w_skout, p.skeys));
  b.soff = static_cast<uint32_t*>(take(f->w_soff, p.soff));
  b.stmp = take(f->w_stmp, p.stmp);
  b.cx = static_cast<float*>(take(f->w_cx, p.cx));
  b.cn = static_cast<float*>(take(f->w_cn, p.cn));
  return b;
}

/// Queries into b.q ([nq][dp], normalized for cosine in b.stage) and, for the MFMA scan, their
/// squared norms into b.qn and their re-score bounds into b.delta; any_delta (nullable, cleared
/// beforehand) is set when some query's bound is not 0. With thr, also the MFMA scan's words:
/// thr_stride prune bounds per query in thr and the fallback count in b.fb.
void flat_prep_queries(qvh_flat* f, const FlatBuffers& b, const float* d_raw, uint64_t nq, hipStream_t s,
                       uint32_t* any_delta = nullptr, uint32_t* thr = nullptr, uint32_t thr_stride = 0) {
  const float* qs = d_raw;
  if (f->metric == QVH_METRIC_COSINE) {  // normalized in a copy
    if (b.stage != d_raw) {
      QVH_HIP(hipMemcpyAsync(b.stage, d_raw, nq * f->dim * sizeof(float), hipMemcpyDeviceToDevice, s));
    }
    launch_normalize_rows(b.stage, nq, f->dim, s);
    qs = b.stage;
  }
  hipLaunchKernelGGL(prep_queries_kernel, dim3(static_cast<unsigned>(ceil_div(nq, 4))), dim3(256), 0, s, qs, b.q, nq,
                     f->dim, f->dp, b.qn, f->meta.as<uint32_t>(), f->metric == QVH_METRIC_L2 ? 1 : 0, b.delta,
                     any_delta, thr != nullptr ? b.fb : nullptr, thr, thr_stride);
  QVH_HIP(hipGetLastError());
}

/// Runs a planned search on its workspace. d_idx (nullable, n_idx entries, ascending) lists the
/// admitted rows for the MFMA scan; the caller passes it instead of the bitmap when few rows are
/// admitted.
void flat_search_run(qvh_flat* f, const FlatPlan& p, const FlatBuffers& b, const float* d_queries, uint64_t nq,
                     uint32_t k, const uint64_t* d_bitmap, uint32_t* d_rows, float* d_dist, hipStream_t s,
                     const uint32_t* d_idx = nullptr, uint64_t n_idx = 0) {
  f->last_fb = p.path == FlatPlan::kMfma;
  f->last_fb_count = b.fb;
  f->timed = f->timing;
  if (f->timed) QVH_HIP(hipEventRecord(f->ev[0], s));
  uint32_t* gate = p.path == FlatPlan::kMfma && p.kl_exact ? b.fb + nq + 1 : nullptr;
  // The launch gate is cleared before the prep raises it; the MFMA scan's other words are set by the
  // prep (its shared bounds, strided for the ring scan, and the fallback count).
  if (gate) hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, s, gate, 1, 0u);
  if (p.path == FlatPlan::kMfma) {
    flat_prep_queries(f, b, d_queries, nq, s, gate, b.thr, p.ring ? kRingBoundStride : kScanBoundStride);
  } else {
    flat_prep_queries(f, b, d_queries, nq, s);
  }
  if (f->timed) QVH_HIP(hipEventRecord(f->ev[1], s));
  ExactArgs e{};
  e.X = f->rows.as<float>();
  e.dp = f->dp;
  e.dim = f->dim;
  e.n = f->n;
  e.Q = b.q;
  e.k = k;
  e.l2 = f->metric == QVH_METRIC_L2;
  e.bitmap = d_bitmap;
  e.out_rows = d_rows;
  e.out_dist = d_dist;
  e.qlist = nullptr;
  e.qcount = nullptr;
  if (p.path == FlatPlan::kSorted) {
    if (d_idx) {
      e.idx = d_idx;
      e.n = n_idx;
      e.bitmap = nullptr;
    }
    run_sorted(SortBuffers{p.sort_chunk, b.skin, b.skout, b.soff, b.stmp, p.stmp}, e, nq, k, s);
    f->last_nsplit = 0;
    if (f->timed) {
      QVH_HIP(hipEventRecord(f->ev[2], s));
      QVH_HIP(hipEventRecord(f->ev[3], s));
    }
    return;
  }
  if (p.path == FlatPlan::kFew) {
    const bool l2 = f->metric == QVH_METRIC_L2;
    const dim3 grid(static_cast<unsigned>(p.g)), block(kFewThreads);
    const bool tail = f->dim % 32 != 0;
    for (uint64_t q0 = 0; q0 < nq; q0 += kFewMaxQ) {
      const uint64_t nc = std::min<uint64_t>(kFewMaxQ, nq - q0);
      FewArgs fa;
      fa.X = f->rows.as<float>();
      fa.dp = f->dp;
      fa.dim = f->dim;
      fa.n = f->n;
      fa.Q = b.q + q0 * f->dp;
      fa.nq = static_cast<uint32_t>(nc);
      fa.k = k;
      fa.bitmap = d_bitmap;
      fa.rows_per_split = p.rps;
      fa.nsplit = static_cast<uint32_t>(p.g);
      fa.part_r = b.pr + q0 * p.g * k;  // [query][split][k]
      fa.part_d = b.pd + q0 * p.g * k;
      auto go = [&](auto nqc) {
        constexpr int NQ = decltype(nqc)::value;
        auto kern = k > 64 ? (l2 ? flat_few_kernel<NQ, true, false, 256> : flat_few_kernel<NQ, false, false, 256>)
                    : l2   ? (tail ? flat_few_kernel<NQ, true, true> : flat_few_kernel<NQ, true, false>)
                           : (tail ? flat_few_kernel<NQ, false, true> : flat_few_kernel<NQ, false, false>);
        hipLaunchKernelGGL(kern, grid, block, 0, s, fa);
      };
      if (nc <= 1) {
        go(std::integral_constant<int, 1>{});
      } else if (nc <= 2) {
        go(std::integral_constant<int, 2>{});
      } else if (nc <= 4) {
        go(std::integral_constant<int, 4>{});
      } else {
        go(std::integral_constant<int, 8>{});
      }
      QVH_HIP(hipGetLastError());
    }
    if (f->timed) QVH_HIP(hipEventRecord(f->ev[2], s));
    launch_sorted_merge(b.pr, b.pd, nq, static_cast<uint32_t>(p.g), k, d_rows, d_dist, b.mflag, s);
    f->last_nsplit = p.g;
    if (f->timed) QVH_HIP(hipEventRecord(f->ev[3], s));
    return;
  }
  if (p.path == FlatPlan::kSplit) {
    e.nsplit = static_cast<uint32_t>(p.g);
    e.nq = static_cast<uint32_t>(nq);
    e.rows_per_split = p.rps;
    e.out_rows = b.pr;
    e.out_dist = b.pd;
    launch_exact(e, nq, s);
    if (f->timed) QVH_HIP(hipEventRecord(f->ev[2], s));
    launch_sorted_merge(b.pr, b.pd, nq, e.nsplit, k, d_rows, d_dist, b.mflag, s);
    f->last_nsplit = p.g;
    if (f->timed) QVH_HIP(hipEventRecord(f->ev[3], s));
    return;
  }
  if (p.path == FlatPlan::kExactOnly) {
    launch_exact(e, nq, s);
    f->last_nsplit = 0;
    if (f->timed) {
      QVH_HIP(hipEventRecord(f->ev[2], s));
      QVH_HIP(hipEventRecord(f->ev[3], s));
    }
    return;
  }
  ScanArgs a;
  a.gate = nullptr;
  a.gate_want = 0;
  a.X = f->rows.as<float>();
  a.xnorm = f->norms.as<float>();
  a.n = p.scan_rows;
  a.Q = b.q;
  a.qnorm = b.qn;
  a.nq = static_cast<uint32_t>(nq);
  a.bitmap = d_idx ? nullptr : d_bitmap;
  a.l2 = f->metric == QVH_METRIC_L2;
  if (d_idx && n_idx > 0) {
    // The listed rows in list order: the scan's positions are positions in the list, which the
    // merge and the fallback map to rows through d_idx.
    QVH_REQUIRE(b.cx != nullptr, "flat search: no workspace for the listed rows");
    const uint64_t chunks = n_idx * (f->dp / 4);
    const unsigned blocks = static_cast<unsigned>(
        std::min<uint64_t>(ceil_div(chunks, 256), static_cast<uint64_t>(device_cus(f->device)) * 16));
    hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks), dim3(256), 0, s, f->rows.as<float>(),
                       a.l2 ? f->norms.as<float>() : nullptr, d_idx, n_idx, f->dp / 4, b.cx, b.cn);
    QVH_HIP(hipGetLastError());
    a.X = b.cx;
    if (a.l2) a.xnorm = b.cn;
  }
  a.nsplit = static_cast<uint32_t>(p.nsplit);
  a.qblocks = p.qblocks;
  a.rows_per_split = p.rows_per_split;
  a.part_d = b.pd;
  a.part_r = b.pr;
  a.qthr = b.thr;
  // The wide merge's R = k + max(16, k / 2) keys: up to R = 64 the register scan shares a bound of
  // rank ceil(R / 2) (1M x 128 integer mixture, 10k queries, k = 32: 28.9 ms with no shared bound).
  const uint32_t wide_sel = k + std::max<uint32_t>(16, k / 2);
  a.share_rank = p.wide && wide_sel <= 64 && f->dp <= static_cast<uint32_t>(kMaxDp) ? (wide_sel + 1) / 2 : 0;
  a.share = !p.wide || a.share_rank != 0 ? 1 : 0;
  a.dp = f->dp;
  // One query block of at most 128 queries, unfiltered, register-resident queries: the row-split
  // form of the scan (two waves per 32-query group).
  a.rowsplit = nq <= static_cast<uint64_t>(kQueriesPerBlock / 2) && !d_idx && !d_bitmap && f->dp <= kMaxDp ? 1 : 0;
  a.bound_slots = !p.wide && (!a.rowsplit || p.nsplit <= kScanSlotMaxSplits) ? 1 : 0;
  const dim3 sgrid(static_cast<unsigned>(p.qblocks * p.nsplit));
  auto scan = [&](int kl) {
    if (p.ring) {
      launch_ring(f->dp, kl, sgrid, a, s);
    } else {
      launch_scan(f->dp, kl, sgrid, a, s);
    }
  };
  if (gate) {  // exact distances for every query: the short lists; otherwise the margin's
    a.gate = gate;
    a.gate_want = 0;
    scan(p.kl_exact);
    a.gate_want = 1;
  }
  scan(p.kl);
  QVH_HIP(hipGetLastError());
  if (f->timed) QVH_HIP(hipEventRecord(f->ev[2], s));
  f->last_nsplit = p.nsplit;

  MergeArgs m;
  m.gate = nullptr;
  m.gate_want = 0;
  m.X = f->rows.as<float>();
  m.dim = f->dim;
  m.dp = f->dp;
  m.Q = a.Q;
  m.nq = a.nq;
  m.k = k;
  m.l2 = a.l2;
  m.nlists = static_cast<uint32_t>(2 * p.nsplit);
  m.part_d = a.part_d;
  m.part_r = a.part_r;
  m.idx = d_idx;
  m.out_rows = d_rows;
  m.out_dist = d_dist;
  m.delta = b.delta;
  // fb[0] counts the queries whose selection the merge could not certify (or, in the wide merge,
  // whose list ran out), fb[1..] lists them; the exact kernel then recomputes only those.
  uint32_t* fb = b.fb;  // reset before the prep
  m.fallback = fb + 1;
  m.nfallback = fb;
  const dim3 mgrid(static_cast<unsigned>(ceil_div(nq, 4)));
  if (p.wide) {
    const uint32_t sel_n = k + std::max<uint32_t>(16, k / 2);
    hipLaunchKernelGGL(flat_merge_wide_kernel, mgrid, dim3(256), 0, s, m, sel_n);
  } else {
    if (gate) {  // the merge of the short lists, or (gate set) of the margin's
      m.gate = gate;
      m.gate_want = 0;
      hipLaunchKernelGGL(flat_merge_kernel<10>, mgrid, dim3(256), 0, s, m);  // exact_list_length
      m.gate_want = 1;
    }
    if (p.kl == 16) {
      hipLaunchKernelGGL(flat_merge_kernel<16>, mgrid, dim3(256), 0, s, m);
    } else {
      hipLaunchKernelGGL(flat_merge_kernel<32>, mgrid, dim3(256), 0, s, m);
    }
  }
  QVH_HIP(hipGetLastError());
  e.qlist = fb + 1;
  e.qcount = fb;
  if (d_idx) {  // positions of the listed rows, as the scan saw them
    e.idx = d_idx;
    e.n = n_idx;
    e.bitmap = nullptr;
  }
  // The first kFallbackSplitQueries listed queries run over row splits (a single work-group per
  // query would read every row alone: 1024-d, 500k rows, three uncertified queries took 112 ms),
  // into the scan's partial lists, which the merge has consumed; the rest one work-group each.
  const uint32_t fsplit = fallback_splits(e.n, device_cus(f->device));
  const size_t part_entries = static_cast<size_t>(nq) * 2 * p.nsplit * p.kl;
  if (k <= 64 && fsplit >= 8 && static_cast<size_t>(kFallbackSplitQueries) * fsplit * k <= part_entries) {
    ExactArgs es = e;
    es.nsplit = fsplit;
    es.nq = kFallbackSplitQueries;
    es.rows_per_split = ceil_div(ceil_div(e.n, fsplit), kExactThreads) * kExactThreads;
    es.out_rows = b.pr;
    es.out_dist = b.pd;
    launch_exact(es, kFallbackSplitQueries, s);
    hipLaunchKernelGGL(flat_merge_select_kernel, dim3(kFallbackSplitQueries), dim3(1024), 0, s, b.pr, b.pd, fsplit, k,
                       d_rows, d_dist, nullptr, fb + 1, fb);
    QVH_HIP(hipGetLastError());
    e.qskip = kFallbackSplitQueries;
  }
  // At most nq queries fall back: with no more than the split form takes, none is left for this.
  if (e.qskip < nq) launch_exact(e, nq, s);
  if (f->timed) QVH_HIP(hipEventRecord(f->ev[3], s));
}

/// A search on the handle's own workspace. d_idx as for flat_search_run.
void flat_search_impl(qvh_flat* f, const float* d_queries, uint64_t nq, uint32_t k,
                      const uint64_t* d_bitmap, uint32_t* d_rows, float* d_dist, hipStream_t s,
                      const uint32_t* d_idx = nullptr, uint64_t n_idx = 0) {
  const FlatPlan p = plan_flat_search(f, nq, k, d_idx != nullptr, d_bitmap != nullptr, n_idx, device_cus(f->device));
  flat_search_run(f, p, handle_buffers(f, p), d_queries, nq, k, d_bitmap, d_rows, d_dist, s, d_idx, n_idx);
}

/// True when a filter of `admitted` rows can run as listed rows: the MFMA scan serves k, and the
/// rows' contiguous copy fits kCompactMaxBytes.
bool listed_scan_applies(const qvh_flat* f, uint32_t k, uint64_t admitted) {
  return shared_list_length(k) != 0 && f->dp <= kMaxChunkedDp && admitted * f->dp * sizeof(float) <= kCompactMaxBytes;
}

/// A caller's list of admitted rows into the handle's copy, each row clamped below n (a row past
/// the store reads the last stored row instead of memory past it).
__global__ void clamp_rows_kernel(const uint32_t* __restrict__ src, uint64_t count, uint64_t n,
                                  uint32_t* __restrict__ dst) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) {
    const uint32_t r = src[i];
    dst[i] = r < n ? r : static_cast<uint32_t>(n - 1);
  }
}

__global__ void zero_words_kernel(uint64_t* __restrict__ p, uint64_t count) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) p[i] = 0;
}

/// Sets the bit of every listed row (below n, as clamp_rows_kernel leaves them) in a cleared bitmap.
__global__ void rows_to_bitmap_kernel(const uint32_t* __restrict__ rows, uint64_t count, uint64_t* bits) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) {
    const uint32_t r = rows[i];
    atomicOr(reinterpret_cast<unsigned long long*>(bits + (r >> 6)), 1ull << (r & 63));
  }
}

}  // namespace

extern "C" {

qvh_status qvh_flat_create(uint32_t dim, int metric, qvh_flat** out) {
  return guarded([&] {
    QVH_REQUIRE(out != nullptr, "qvh_flat_create: null output");
    *out = nullptr;
    QVH_REQUIRE(dim >= 1 && dim <= 65536, "dimension must be in [1, 65536]");
    QVH_REQUIRE(metric >= QVH_METRIC_L2 && metric <= QVH_METRIC_COSINE, "unknown metric");
    const uint32_t dp = padded_dim(dim);
    const int dev = current_device();
    auto* f = new qvh_flat;
    f->dim = dim;
    f->dp = dp;
    f->metric = metric;
    f->device = dev;
    const hipError_t e = hipStreamCreateWithFlags(&f->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete f;
      throw Failure(QVH_EDEVICE, std::string("hipStreamCreate: ") + hipGetErrorString(e));
    }
    try {
      f->meta.reserve(2 * sizeof(uint32_t));
      hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, f->stream, f->meta.as<uint32_t>(), 2, 0u);
      QVH_HIP(hipGetLastError());
      // Created here rather than on the first call from another stream, so that the search
      // without allocation never creates one.
      QVH_HIP(hipEventCreateWithFlags(&f->join, hipEventDisableTiming));
      QVH_HIP(hipStreamSynchronize(f->stream));
    } catch (...) {
      qvh_flat_destroy(f);
      throw;
    }
    *out = f;
  });
}

void qvh_flat_destroy(qvh_flat* f) {
  if (!f) return;
  (void)hipSetDevice(f->device);
  if (f->stream) {
    (void)hipStreamSynchronize(f->stream);
    (void)hipStreamDestroy(f->stream);
  }
  for (hipEvent_t& e : f->ev) {
    if (e) (void)hipEventDestroy(e);
  }
  if (f->join) (void)hipEventDestroy(f->join);
  delete f;
}

qvh_status qvh_flat_set_timing(qvh_flat* f, int enable) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr, "qvh_flat_set_timing: null handle");
    std::lock_guard<std::mutex> lock(f->mu);
    QVH_HIP(hipSetDevice(f->device));
    if (enable && !f->ev[0]) {
      for (hipEvent_t& e : f->ev) QVH_HIP(hipEventCreate(&e));
    }
    f->timing = enable != 0;
  });
}

qvh_status qvh_flat_last_fallbacks(qvh_flat* f, uint32_t* count) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr && count != nullptr, "qvh_flat_last_fallbacks: null argument");
    std::lock_guard<std::mutex> lock(f->mu);
    QVH_HIP(hipSetDevice(f->device));
    *count = 0;
    if (!f->last_fb) return;
    QVH_HIP(hipStreamSynchronize(f->stream));
    QVH_HIP(hipMemcpy(count, f->last_fb_count, sizeof(uint32_t), hipMemcpyDeviceToHost));
  });
}

qvh_status qvh_flat_last_timing(qvh_flat* f, float* prep_ms, float* scan_ms, float* merge_ms,
                                uint32_t* nsplit) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr, "qvh_flat_last_timing: null handle");
    std::lock_guard<std::mutex> lock(f->mu);
    QVH_REQUIRE(f->timed, "qvh_flat_last_timing: the last search was not timed");
    QVH_HIP(hipSetDevice(f->device));
    QVH_HIP(hipEventSynchronize(f->ev[3]));
    float t[3];
    for (int i = 0; i < 3; ++i) QVH_HIP(hipEventElapsedTime(&t[i], f->ev[i], f->ev[i + 1]));
    if (prep_ms) *prep_ms = t[0];
    if (scan_ms) *scan_ms = t[1];
    if (merge_ms) *merge_ms = t[2];
    if (nsplit) *nsplit = static_cast<uint32_t>(f->last_nsplit);
  });
}

uint64_t qvh_flat_size(const qvh_flat* f) { return f ? f->n : 0; }

namespace {

void flat_append(qvh_flat* f, const float* rows, uint64_t n, float* stored_out, bool as_stored) {
  QVH_REQUIRE(f != nullptr, "qvh_flat_append: null handle");
  if (n == 0) return;
  QVH_REQUIRE(rows != nullptr, "qvh_flat_append: null rows");
  std::lock_guard<std::mutex> lock(f->mu);
  QVH_REQUIRE(f->n + n <= 0xFFFFFFFFull, "FlatIndex holds at most 2^32 vectors");
  QVH_HIP(hipSetDevice(f->device));
  flat_grow(f, f->n + n);
  const size_t raw_bytes = n * f->dim * sizeof(float);
  float* stage = static_cast<float*>(f->w_stage.reserve(raw_bytes));
  QVH_HIP(hipMemcpyAsync(stage, rows, raw_bytes, hipMemcpyHostToDevice, f->stream));
  if (f->metric == QVH_METRIC_COSINE && !as_stored) launch_normalize_rows(stage, n, f->dim, f->stream);
  float* dst = f->rows.as<float>() + f->n * f->dp;
  const uint64_t total = n * f->dp;
  hipLaunchKernelGGL(pack_rows_kernel, dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256), 0,
                     f->stream, stage, dst, n, f->dim, f->dp);
  hipLaunchKernelGGL(row_norms_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0,
                     f->stream, dst, f->norms.as<float>() + f->n, n, f->dp, f->meta.as<uint32_t>());
  QVH_HIP(hipGetLastError());
  QVH_HIP(hipMemcpyAsync(f->h_meta, f->meta.ptr, sizeof(f->h_meta), hipMemcpyDeviceToHost, f->stream));
  if (stored_out) QVH_HIP(hipMemcpyAsync(stored_out, stage, raw_bytes, hipMemcpyDeviceToHost, f->stream));
  QVH_HIP(hipStreamSynchronize(f->stream));
  f->n += n;
  float top;  // largest stored squared norm
  std::memcpy(&top, &f->h_meta[0], sizeof(top));
  f->integral_rows = f->h_meta[1] == 0 && top <= 16777216.0f;
}

}  // namespace

qvh_status qvh_flat_append(qvh_flat* f, const float* rows, uint64_t n, float* stored_out) {
  return guarded([&] { flat_append(f, rows, n, stored_out, false); });
}

qvh_status qvh_flat_append_stored(qvh_flat* f, const float* rows, uint64_t n) {
  return guarded([&] { flat_append(f, rows, n, nullptr, true); });
}

qvh_status qvh_flat_search(qvh_flat* f, const float* queries, uint64_t nq, uint32_t k,
                           const uint64_t* row_bitmap, uint32_t* out_rows, float* out_dist) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr, "qvh_flat_search: null handle");
    if (nq == 0 || k == 0) return;
    QVH_REQUIRE(queries && out_rows && out_dist, "qvh_flat_search: null buffer");
    std::lock_guard<std::mutex> lock(f->mu);
    QVH_HIP(hipSetDevice(f->device));
    const size_t qbytes = nq * f->dim * sizeof(float);
    float* d_raw = static_cast<float*>(f->w_stage.reserve(qbytes));
    QVH_HIP(hipMemcpyAsync(d_raw, queries, qbytes, hipMemcpyHostToDevice, f->stream));
    const uint64_t* d_bits = nullptr;
    const uint32_t* d_idx = nullptr;
    std::vector<uint32_t> listed;
    if (row_bitmap) {
      const size_t words = ceil_div(std::max<uint64_t>(f->n, 1), 64);
      // The admitted rows, counted.
      uint64_t admitted = 0;
      for (size_t w = 0; w < words; ++w) {
        uint64_t bits = row_bitmap[w];
        if (w + 1 == words && f->n % 64) bits &= (1ull << (f->n % 64)) - 1;
        admitted += static_cast<uint64_t>(__builtin_popcountll(bits));
      }
      // A filter that admits every row is no filter. Any other goes to the MFMA scan as the list of
      // its rows while their contiguous copy fits: the scan then reads only admitted rows, where
      // the bitmap form reads every row and tests it (1.18M x 100 cosine, 10,000 queries: 55% of
      // the rows admitted 23.8 ms as a bitmap, 90% 23.8 ms, none filtered 21.0 ms; listed rows
      // run in proportion to their count, 45% in 10.3 ms).
      if (admitted == f->n) {
        row_bitmap = nullptr;
      } else if (listed_scan_applies(f, k, admitted)) {
        listed.reserve(admitted);
        for (size_t w = 0; w < words; ++w) {
          uint64_t bits = row_bitmap[w];
          if (w + 1 == words && f->n % 64) bits &= (1ull << (f->n % 64)) - 1;
          while (bits) {
            listed.push_back(static_cast<uint32_t>(w * 64 + static_cast<uint64_t>(__builtin_ctzll(bits))));
            bits &= bits - 1;
          }
        }
        uint32_t* li = static_cast<uint32_t*>(f->w_idx.reserve(std::max<size_t>(listed.size(), 1) * sizeof(uint32_t)));
        if (!listed.empty()) {
          QVH_HIP(hipMemcpyAsync(li, listed.data(), listed.size() * sizeof(uint32_t), hipMemcpyHostToDevice, f->stream));
        }
        d_idx = li;
      } else {
        uint64_t* b = static_cast<uint64_t*>(f->w_bits.reserve(words * sizeof(uint64_t)));
        QVH_HIP(hipMemcpyAsync(b, row_bitmap, words * sizeof(uint64_t), hipMemcpyHostToDevice, f->stream));
        d_bits = b;
      }
    }
    uint32_t* d_rows = static_cast<uint32_t*>(f->w_rows.reserve(nq * k * sizeof(uint32_t)));
    float* d_dist = static_cast<float*>(f->w_dist.reserve(nq * k * sizeof(float)));
    flat_search_impl(f, d_raw, nq, k, d_bits, d_rows, d_dist, f->stream, d_idx, listed.size());
    QVH_HIP(hipMemcpyAsync(out_rows, d_rows, nq * k * sizeof(uint32_t), hipMemcpyDeviceToHost, f->stream));
    QVH_HIP(hipMemcpyAsync(out_dist, d_dist, nq * k * sizeof(float), hipMemcpyDeviceToHost, f->stream));
    QVH_HIP(hipStreamSynchronize(f->stream));
  });
}

qvh_status qvh_flat_search_rows(qvh_flat* f, const float* queries, uint64_t nq, uint32_t k,
                                const uint32_t* rows, uint64_t nrows, uint32_t* out_rows, float* out_dist) {
  std::vector<uint64_t> bits;
  {
    const qvh_status st = guarded([&] {
      QVH_REQUIRE(f != nullptr, "qvh_flat_search_rows: null handle");
      QVH_REQUIRE(rows != nullptr || nrows == 0, "qvh_flat_search_rows: null rows");
      uint64_t n = 0;
      {
        std::lock_guard<std::mutex> lock(f->mu);
        n = f->n;
      }
      // The listed rows as a row bitmap: the same admitted set as a filter over their labels.
      bits.assign(ceil_div(std::max<uint64_t>(n, 1), 64), 0);
      for (uint64_t i = 0; i < nrows; ++i) {
        QVH_REQUIRE(rows[i] < n, "qvh_flat_search_rows: row " + std::to_string(rows[i]) + " is not stored");
        bits[rows[i] >> 6] |= 1ull << (rows[i] & 63);
      }
    });
    if (st != QVH_OK) return st;
  }
  return qvh_flat_search(f, queries, nq, k, bits.data(), out_rows, out_dist);
}

qvh_status qvh_flat_search_device(qvh_flat* f, const float* d_queries, uint64_t nq, uint32_t k,
                                  const uint64_t* d_row_bitmap, uint32_t* d_out_rows,
                                  float* d_out_dist, void* stream) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr, "qvh_flat_search_device: null handle");
    if (nq == 0 || k == 0) return;
    QVH_REQUIRE(d_queries && d_out_rows && d_out_dist, "qvh_flat_search_device: null buffer");
    std::lock_guard<std::mutex> lock(f->mu);
    QVH_HIP(hipSetDevice(f->device));
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : f->stream;
    on_handle_timeline(f->stream, f->join, s, [&](hipStream_t st) {
      flat_search_impl(f, d_queries, nq, k, d_row_bitmap, d_out_rows, d_out_dist, st);
    });
  });
}

qvh_status qvh_flat_search_device_rows(qvh_flat* f, const float* d_queries, uint64_t nq, uint32_t k,
                                       const uint32_t* d_row_list, uint64_t nrows, uint32_t* d_out_rows,
                                       float* d_out_dist, void* stream) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr, "qvh_flat_search_device_rows: null handle");
    if (nq == 0 || k == 0) return;
    QVH_REQUIRE(d_queries && d_out_rows && d_out_dist, "qvh_flat_search_device_rows: null buffer");
    QVH_REQUIRE(d_row_list != nullptr || nrows == 0, "qvh_flat_search_device_rows: null row list");
    std::lock_guard<std::mutex> lock(f->mu);
    QVH_REQUIRE(nrows <= f->n, "qvh_flat_search_device_rows: " + std::to_string(nrows) + " listed rows but " +
                                   std::to_string(f->n) + " stored");
    QVH_HIP(hipSetDevice(f->device));
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : f->stream;
    on_handle_timeline(f->stream, f->join, s, [&](hipStream_t st) {
      if (nrows == f->n) {  // every stored row listed: no filter
        flat_search_impl(f, d_queries, nq, k, nullptr, d_out_rows, d_out_dist, st);
        return;
      }
      uint32_t* li = static_cast<uint32_t*>(f->w_idx.reserve(std::max<uint64_t>(nrows, 1) * sizeof(uint32_t)));
      if (nrows > 0) {
        hipLaunchKernelGGL(clamp_rows_kernel, dim3(static_cast<unsigned>(ceil_div(nrows, 256))), dim3(256), 0, st,
                           d_row_list, nrows, f->n, li);
        QVH_HIP(hipGetLastError());
      }
      if (listed_scan_applies(f, k, nrows)) {
        flat_search_impl(f, d_queries, nq, k, nullptr, d_out_rows, d_out_dist, st, li, nrows);
        return;
      }
      // The scan over every row with the list as a bitmap.
      const uint64_t words = ceil_div(std::max<uint64_t>(f->n, 1), 64);
      uint64_t* b = static_cast<uint64_t*>(f->w_bits.reserve(words * sizeof(uint64_t)));
      hipLaunchKernelGGL(zero_words_kernel, dim3(static_cast<unsigned>(ceil_div(words, 256))), dim3(256), 0, st, b,
                         words);
      if (nrows > 0) {
        hipLaunchKernelGGL(rows_to_bitmap_kernel, dim3(static_cast<unsigned>(ceil_div(nrows, 256))), dim3(256), 0, st,
                           li, nrows, b);
      }
      QVH_HIP(hipGetLastError());
      flat_search_impl(f, d_queries, nq, k, b, d_out_rows, d_out_dist, st);
    });
  });
}

}  // extern "C"

// ---- search without allocation ------------------------------------------------------------------
//
// qvh_flat_search_device_noalloc takes every buffer beyond its inputs and outputs (prepared queries,
// norms, bounds, partial lists, counters) from `scratch`, a fixed array in device memory that each
// GPU the library runs on holds until the process ends. Its device address on the current device
// comes from hipGetSymbolAddress on the first call there (the name `scratch` is a host-side
// stand-in, not a device address). All calls on one GPU share that GPU's array. The library orders
// them on the device: each call's stream first waits for an event the previous call recorded after
// its last launch (a host lock keeps the wait, the launches and the record of concurrent callers
// apart), so calls on different handles or streams take the array in turn. Event waits allocate
// nothing. Under HIP graph capture the calls are not ordered by the library (an event recorded
// outside the graph cannot be waited on inside it): a caller that captures such calls orders its
// replays itself. Every call clears what must start at zero (bounds, counters) itself.

constexpr size_t kScratchBytes = size_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;

/// One device's scratch array: its address, the event its last user recorded, and the lock under
/// which a call waits on that event, launches and records it.
struct ScratchSlot {
  void* ptr = nullptr;
  hipEvent_t done = nullptr;
  bool recorded = false;
  std::mutex use;
};

std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxScratchDevices];

/// The scratch slot of `device`, which must be the current device; its address and event are set up
/// on the first call there.
ScratchSlot& scratch_on(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  QVH_REQUIRE(device >= 0 && device < kMaxScratchDevices, "device index out of range for the scratch array");
  ScratchSlot& slot = g_scratch[device];
  if (slot.ptr == nullptr) {
    void* ptr = nullptr;
    QVH_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    QVH_REQUIRE(ptr != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
    QVH_HIP(hipEventCreateWithFlags(&slot.done, hipEventDisableTiming));
    slot.ptr = ptr;
  }
  return slot;
}

/// The plan's workspace carved from the scratch array, each buffer 256-byte aligned.
FlatBuffers scratch_buffers(unsigned char* base, const FlatPlan& p) {
  size_t at = 0;
  auto take = [&](size_t bytes) -> void* {
    if (bytes == 0) return nullptr;
    void* out = base + at;
    at += FlatPlan::aligned(bytes);
    return out;
  };
  FlatBuffers b;
  b.stage = static_cast<float*>(take(p.stage));
  b.q = static_cast<float*>(take(p.q));
  b.qn = static_cast<float*>(take(p.qn));
  b.delta = static_cast<float*>(take(p.delta));
  b.pd = static_cast<float*>(take(p.pd));
  b.pr = static_cast<uint32_t*>(take(p.pr));
  b.thr = static_cast<uint32_t*>(take(p.thr));
  b.fb = static_cast<uint32_t*>(take(p.fb));
  b.mflag = static_cast<uint32_t*>(take(p.mflag));
  b.skin = static_cast<uint64_t*>(take(p.skeys));
  b.skout = static_cast<uint64_t*>(take(p.skeys));
  b.soff = static_cast<uint32_t*>(take(p.soff));
  b.stmp = take(p.stmp);
  b.cx = static_cast<float*>(take(p.cx));
  b.cn = static_cast<float*>(take(p.cn));
  return b;
}

}  // namespace

extern "C" {

qvh_status qvh_flat_search_device_noalloc(qvh_flat* f, const float* d_queries, uint64_t nq, uint32_t k,
                                          const uint64_t* d_row_bitmap, uint32_t* d_out_rows, float* d_out_dist,
                                          void* stream) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr, "qvh_flat_search_device_noalloc: null handle");
    if (nq == 0 || k == 0) return;
    QVH_REQUIRE(d_queries && d_out_rows && d_out_dist, "qvh_flat_search_device_noalloc: null buffer");
    std::lock_guard<std::mutex> lock(f->mu);
    QVH_HIP(hipSetDevice(f->device));
    ScratchSlot& slot = scratch_on(f->device);
    std::lock_guard<std::mutex> use(slot.use);  // after the handle's lock, never before it
    unsigned char* base = static_cast<unsigned char*>(slot.ptr);
    const FlatPlan p = plan_flat_search(f, nq, k, false, d_row_bitmap != nullptr, 0, device_cus(f->device));
    if (p.total() > kScratchBytes) {
      throw Failure(QVH_EINVAL, "qvh_flat_search_device_noalloc: this search needs " + std::to_string(p.total()) +
                                    " bytes of workspace, above the fixed scratch of " +
                                    std::to_string(kScratchBytes) + " bytes; search fewer queries per call");
    }
    const FlatBuffers b = scratch_buffers(base, p);
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : f->stream;
    on_handle_timeline(f->stream, f->join, s, [&](hipStream_t st) {
      hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
      QVH_HIP(hipStreamIsCapturing(st, &capture));
      const bool ordered = capture == hipStreamCaptureStatusNone;
      if (ordered && slot.recorded) QVH_HIP(hipStreamWaitEvent(st, slot.done, 0));
      flat_search_run(f, p, b, d_queries, nq, k, d_row_bitmap, d_out_rows, d_out_dist, st);
      if (ordered) {
        QVH_HIP(hipEventRecord(slot.done, st));
        slot.recorded = true;
      }
    });
  });
}

qvh_status qvh_flat_sync(qvh_flat* f) {
  return guarded([&] {
    QVH_REQUIRE(f != nullptr, "qvh_flat_sync: null handle");
    QVH_HIP(hipSetDevice(f->device));
    QVH_HIP(hipStreamSynchronize(f->stream));
  });
}

}  // extern "C"
