// IVF-PQ on gfx950: batched encode on add (IvfPqIndex::Impl::add, src/ivfpq_index.cc:208-271) and
// the query path of IvfPqIndex::Impl::search_into (src/ivfpq_index.cc:275-381).
//
// Device layout (one handle):
//   centroids   [nlist][dim] and transposed [dim][nlist]; ||c||^2 per centroid
//   codebook    [m][256][dsub] and, per sub-space, transposed [m][dsub][256]
//   precomputed [nlist][m][256] (L2 only, when it fits the reference's 256 MiB budget)
//   lists in CSR order: offsets [nlist+1] (u64), codes [count][mp] (u8, mp = m rounded up to 4),
//   term1 [count] (L2 precomputed: sum_j pre[l][j][code_j]), vectors [count][dim] (store_vectors)
// Labels stay on the host; the device speaks of CSR positions and refs (list << 32 | offset).
//
// Arithmetic: assignment, PQ codes, coarse scores, the precomputed table, the per-query tables and
// the ADC sums replay the reference's unfused, in-order float operations (all qvh sources are
// compiled with -ffp-contract=off), so codes and assignments are bit-identical. For L2 with the
// precomputed table the scan ranks candidates by base + term1 + sum_j qtab[j][c_j] (the same
// quantity, grouped differently), then re-scores the best keep + margin candidates exactly as the
// reference adds them (base + sum_j (pre[l][j][c_j] + qtab[j][c_j])).
#include <algorithm>
#include <atomic>
#include <cstring>
#include <numeric>
#include <vector>

#include "common.hpp"
#include "exact.hpp"
#include "select.hpp"

namespace qvh {
void launch_normalize_rows(float* d_rows, uint64_t n, uint32_t dim, hipStream_t stream);
}

namespace {

using namespace qvh;

constexpr int kModePre = 0;       // L2 with precomputed table (approximate scan + exact re-score)
constexpr int kModeIp = 1;        // inner product / cosine: exact scan
constexpr int kModeResidual = 2;  // L2 without precomputed table: per-list residual tables, exact

// ---- exact nearest centroid / PQ encode -------------------------------------------------------

constexpr int kNearThreads = 256;
constexpr int kNearCT = 64;  // centroids per tile (accumulators per thread)
constexpr int kNearJC = 32;  // dims per staged chunk

struct NearestArgs {
  const float* x;        // point p, dim t at x[p * x_stride + x_off + t]
  uint64_t n;
  uint32_t dim;
  uint64_t x_stride;
  uint32_t x_off;
  const float* ct;       // transposed centroids [dim][k] (for the sub-space: + sub * dim * k)
  const float* norms;    // [k] ||c||^2 (nearest mode)
  uint32_t k;
  int max_ip;
  uint32_t* out32;       // nearest mode: out32[p]
  uint8_t* out8;         // sqdiff mode: out8[p * out_stride + sub]
  uint32_t out_stride;
  const uint32_t* list;  // if set: the points list[1 .. list[0]] only (nearest mode)
};

/// SQDIFF = false: CentroidTable::nearest_batch (src/internal/centroid_table.h:94-144):
///   dot_c = sum_j x_j * c_j in order of j, d_c = max_ip ? -dot_c : ||c||^2 - 2 dot_c, first strictly
///   smaller wins, 0 if every d_c is NaN.
/// SQDIFF = true: CentroidTable::l2 + argmin_n (centroid_table.h:65-75,155-170) for PQ encode:
///   d_c = sum_t (x_t - c_t)^2 in order of t; the first index holding the minimum over the non-NaN
///   values; 0 if there is none. blockIdx.y is the sub-space.
template <bool SQDIFF>
__global__ void __launch_bounds__(kNearThreads) nearest_kernel(NearestArgs a) {
  __shared__ float s_x[kNearJC][kNearThreads];
  __shared__ __attribute__((aligned(16))) float s_c[kNearJC][kNearCT];
  const int tid = threadIdx.x;
  uint64_t p = static_cast<uint64_t>(blockIdx.x) * kNearThreads + tid;
  const uint32_t sub = blockIdx.y;
  bool valid = p < a.n;
  if (a.list) {
    // The grid covers every point; blocks past the listed count leave before any barrier.
    const uint32_t cnt = a.list[0];
    if (static_cast<uint64_t>(blockIdx.x) * kNearThreads >= cnt) return;
    valid = p < cnt;
    p = valid ? a.list[1 + p] : 0;
  }
  const uint64_t prow = valid ? p : 0;
  const float* xrow = a.x + prow * a.x_stride + a.x_off + static_cast<uint64_t>(sub) * a.dim;
  const float* ct = a.ct + static_cast<uint64_t>(sub) * a.dim * a.k;

  float best = __builtin_huge_valf();
  int64_t arg = -1;
  for (uint32_t c0 = 0; c0 < a.k; c0 += kNearCT) {
    float acc[kNearCT];
#pragma unroll
    for (int c = 0; c < kNearCT; ++c) acc[c] = 0.0f;
    for (uint32_t j0 = 0; j0 < a.dim; j0 += kNearJC) {
      const uint32_t jn = min(static_cast<uint32_t>(kNearJC), a.dim - j0);
      __syncthreads();
      for (uint32_t jj = 0; jj < jn; ++jj) s_x[jj][tid] = xrow[j0 + jj];
      for (uint32_t e = tid; e < jn * kNearCT; e += kNearThreads) {
        const uint32_t jj = e / kNearCT, c = e % kNearCT;
        s_c[jj][c] = c0 + c < a.k ? ct[static_cast<uint64_t>(j0 + jj) * a.k + c0 + c] : 0.0f;
      }
      __syncthreads();
      for (uint32_t jj = 0; jj < jn; ++jj) {
        const float xv = s_x[jj][tid];
#pragma unroll
        for (int c = 0; c < kNearCT; c += 4) {
          const float4 cv = *reinterpret_cast<const float4*>(&s_c[jj][c]);
          if constexpr (SQDIFF) {
            const float d0 = xv - cv.x, d1 = xv - cv.y, d2 = xv - cv.z, d3 = xv - cv.w;
            acc[c + 0] = acc[c + 0] + d0 * d0;
            acc[c + 1] = acc[c + 1] + d1 * d1;
            acc[c + 2] = acc[c + 2] + d2 * d2;
            acc[c + 3] = acc[c + 3] + d3 * d3;
          } else {
            acc[c + 0] = acc[c + 0] + xv * cv.x;
            acc[c + 1] = acc[c + 1] + xv * cv.y;
            acc[c + 2] = acc[c + 2] + xv * cv.z;
            acc[c + 3] = acc[c + 3] + xv * cv.w;
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < kNearCT; ++c) {
      if (c0 + c < a.k) {
        float d;
        if constexpr (SQDIFF) {
          d = acc[c];
          // argmin_n: strictly smaller wins; the first +inf counts when nothing finite came first
          if (d < best || (arg < 0 && d == best)) {
            best = d;
            arg = c0 + c;
          }
        } else {
          d = a.max_ip ? -acc[c] : a.norms[c0 + c] - 2.0f * acc[c];
          if (d < best) {
            best = d;
            arg = c0 + c;
          }
        }
      }
    }
  }
  if (!valid) return;
  const uint32_t r = arg < 0 ? 0u : static_cast<uint32_t>(arg);
  if constexpr (SQDIFF) {
    a.out8[p * a.out_stride + sub] = static_cast<uint8_t>(r);
  } else {
    a.out32[p] = r;
  }
}


// ---- MFMA assignment with a certificate -------------------------------------------------------
//
// CentroidTable::nearest_batch (src/internal/centroid_table.h:94-144) for many points: the matrix
// unit computes g_c = ||c||^2 - 2<x,c> (or -<x,c>) for every centroid, the point entering as the
// B operand scaled by -2 (or -1, both exact) and one more MFMA step adding the augmented column
// (||c||^2, or 0; +inf for padding rows). With |g_c - e_c| <= delta for the reference's in-order
// value e_c, only centroids with g_c <= best + 2 delta can be the reference's answer (any other c
// has e_c >= g_c - delta > best + delta >= e_best). Each point keeps its kAsgList smallest (g, c),
// admitting only candidates within 2 delta of its running best (the best only decreases, so the
// others cannot join the final band). When the list's last entry lies above the band, the band's
// members are all in the list: a single member is the answer, and two or more are re-scored in the
// reference's own order and arithmetic. A list whose last entry is inside the band leaves the point
// to the exact kernel. delta = (4(dp + 1) + 16) u (P + R)^2 for L2 and (4(dp + 1) + 16) u P R for
// the inner product, P = ||x||, R = the largest ||c||: the bound on two differently ordered float
// sums of terms whose absolute values add up to at most (P + R)^2 (resp. P R), with a factor of two
// over the derivation for the norms' own rounding and a faithfully rounding matrix unit.

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kAsgThreads = 512;  // 8 waves of 32 points
constexpr int kAsgPoints = 256;
constexpr int kAsgTile = 64;      // centroid rows per LDS tile
constexpr uint32_t kAsgMaxDp = 128;
constexpr uint32_t kAsgMinDim = 32;
constexpr uint64_t kAsgMinPoints = 1024;  // smaller batches stay on the exact kernel
constexpr int kAsgList = 8;                // (g, c) kept per point

/// Inserts (g, c) into the ascending (g, c)-ordered list, dropping the last.
template <int L>
__device__ __forceinline__ void asg_insert(float (&lg)[L], uint32_t (&lc)[L], float g, uint32_t c) {
#pragma unroll
  for (int x = 0; x < L; ++x) {
    const bool lt = (g < lg[x]) | ((g == lg[x]) & (c < lc[x]));
    const float tg = lg[x];
    const uint32_t tc = lc[x];
    lg[x] = lt ? g : tg;
    lc[x] = lt ? c : tc;
    g = lt ? tg : g;
    c = lt ? tc : c;
  }
}

struct AssignArgs {
  const float* x;        // point p at x[p * x_stride], dim floats, 16-byte aligned rows
  uint64_t n;
  uint32_t dim;
  uint64_t x_stride;
  const float* crow;     // [kp][dp] centroid rows, zero-padded
  const float* aug;      // [kp] ||c||^2 (L2) or 0 (inner product); +inf for padding rows
  uint32_t kp;           // rows of crow, a multiple of kAsgTile
  const float* rmax;     // [1] the largest ||c||
  float coef;            // (4 (dp + 1) + 16) * 2^-24
  uint32_t* out32;       // out32[p] for the certified points
  uint32_t* fb;          // fb[0] count, fb[1 + i]: points left to the exact kernel
};

template <int DP, bool L2>
__global__ void __launch_bounds__(kAsgThreads) assign_mfma_kernel(AssignArgs a) {
  constexpr int H = DP / 2;  // dims per lane half
  constexpr int STRIDE = DP + 4;
  constexpr int C4 = DP / 4;
  constexpr int CHUNKS = kAsgTile * C4;
  constexpr int PER_THREAD = (CHUNKS + kAsgThreads - 1) / kAsgThreads;
  __shared__ __attribute__((aligned(16))) float s_tile[2][kAsgTile * STRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const uint64_t p0 = static_cast<uint64_t>(blockIdx.x) * kAsgPoints + wave * 32;
  const uint64_t p = p0 + j;
  const bool wave_active = p0 < a.n;
  const bool valid = p < a.n;

  // Point operand (B, lane = (k = h, col = j)): dims [h*H, h*H + H), scaled.
  constexpr float kScale = L2 ? -2.0f : -1.0f;
  float qreg[H];
  float pp = 0.0f;
  {
    const float* xr = a.x + (valid ? p : 0) * a.x_stride;
#pragma unroll
    for (int s = 0; s < H / 4; ++s) {
      const uint32_t d0 = static_cast<uint32_t>(h * H + 4 * s);
      const f32x4 v = valid && d0 < a.dim ? *reinterpret_cast<const f32x4*>(xr + d0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qreg[4 * s + e] = kScale * v[e];
        pp = pp + v[e] * v[e];
      }
    }
  }
  const float p2 = pp + __shfl_xor(pp, 32, 64);
  const float qaug = h == 0 ? 1.0f : 0.0f;
  const float P = sqrtf(p2), R = a.rmax[0];
  const float delta = L2 ? a.coef * (P + R) * (P + R) : a.coef * P * R;

  const uint32_t ntiles = a.kp / kAsgTile;
  f32x4 stage[PER_THREAD];
  float stage_aug = 0.0f;
  auto load_tile = [&](uint32_t t) {
    const float* base = a.crow + static_cast<uint64_t>(t) * kAsgTile * DP;
#pragma unroll
    for (int pi = 0; pi < PER_THREAD; ++pi) {
      int c = tid + pi * kAsgThreads;
      if (CHUNKS % kAsgThreads != 0) c = c < CHUNKS ? c : CHUNKS - 1;
      stage[pi] = *reinterpret_cast<const f32x4*>(base + (c / C4) * DP + 4 * (c % C4));
    }
    stage_aug = a.aug[static_cast<uint64_t>(t) * kAsgTile + (tid & (kAsgTile - 1))];
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int pi = 0; pi < PER_THREAD; ++pi) {
      const int c = tid + pi * kAsgThreads;
      if (c < CHUNKS) *reinterpret_cast<f32x4*>(&s_tile[buf][(c / C4) * STRIDE + 4 * (c % C4)]) = stage[pi];
    }
    // Column DP + 1 meets the zero of the point's second augmented slot: it must be finite.
    if (tid < kAsgTile) *reinterpret_cast<f32x2*>(&s_tile[buf][tid * STRIDE + DP]) = f32x2{stage_aug, 0.0f};
  };

  float lg[kAsgList];
  uint32_t lc[kAsgList];
#pragma unroll
  for (int x = 0; x < kAsgList; ++x) {
    lg[x] = __builtin_huge_valf();
    lc[x] = 0xFFFFFFFFu;
  }
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (uint32_t t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool prefetch = t + 1 < ntiles;
    if (!wave_active && prefetch) load_tile(t + 1);
    if (wave_active) {
      f32x16 acc0 = {}, acc1 = {};
      const float* r0 = &s_tile[buf][j * STRIDE + h * H];
      const float* r1 = &s_tile[buf][(32 + j) * STRIDE + h * H];
      const float aug0 = s_tile[buf][j * STRIDE + DP + h];
      const float aug1 = s_tile[buf][(32 + j) * STRIDE + DP + h];
      f32x4 x0 = *reinterpret_cast<const f32x4*>(r0);
      f32x4 x1 = *reinterpret_cast<const f32x4*>(r1);
#pragma unroll
      for (int s = 0; s < H; s += 4) {
        f32x4 n0 = x0, n1 = x1;
        if (s + 4 < H) {
          n0 = *reinterpret_cast<const f32x4*>(r0 + s + 4);
          n1 = *reinterpret_cast<const f32x4*>(r1 + s + 4);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[e], qreg[s + e], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[e], qreg[s + e], acc1, 0, 0, 0);
        }
        x0 = n0;
        x1 = n1;
        __builtin_amdgcn_sched_barrier(0);
        if (s == 4 && prefetch) load_tile(t + 1);
        if (s == 4) __builtin_amdgcn_sched_barrier(0);
      }
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(aug0, qaug, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(aug1, qaug, acc1, 0, 0, 0);
      // D[row][col]: col = point j, row = 8*(r/4) + 4*h + r%4 in register r; a lane visits its
      // centroids in increasing order, so a tie with the list's last entry never enters.
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        const f32x16 acc = blk ? acc1 : acc0;
        float mn = acc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mn = fminf(mn, acc[r]);
        // Above the current best + 2 delta a centroid can never join the final band (the best only
        // decreases), so it need not enter the list either.
        const float lim = fminf(lg[kAsgList - 1], lg[0] + 2.0f * delta);
        if (mn < lim) {  // NaN never enters
          const uint32_t cb = t * kAsgTile + 32 * blk + 4 * h;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if (acc[r] < fminf(lg[kAsgList - 1], lg[0] + 2.0f * delta)) {
              asg_insert<kAsgList>(lg, lc, acc[r], cb + 8 * (r >> 2) + (r & 3));
            }
          }
        }
      }
    }
    if (prefetch) store_tile(buf ^ 1);
    __syncthreads();
  }

  // The two lanes of a point saw disjoint centroids: the list of the point is the kAsgList
  // smallest (g, c) of the union of theirs.
  {
    float og[kAsgList];
    uint32_t oc[kAsgList];
#pragma unroll
    for (int x = 0; x < kAsgList; ++x) {
      og[x] = __shfl_xor(lg[x], 32, 64);
      oc[x] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(lc[x]), 32, 64));
    }
#pragma unroll
    for (int x = 0; x < kAsgList; ++x) asg_insert<kAsgList>(lg, lc, og[x], oc[x]);
  }
  // Both lanes of a point hold the same list from here on and decide alike; lane h = 1 writes.
  const float band = lg[0] + 2.0f * delta;
  const bool listed = valid && lg[0] < __builtin_huge_valf() && !(lg[kAsgList - 1] <= band);
  // Exact values of the band's members (a prefix of the list) when there are two or more, in the
  // reference's order and arithmetic: dot = sum_t x_t * c_t from t = 0 (lane h = 0 sums its half,
  // lane h = 1 continues from that partial sum; the zero padding adds +0), then ||c||^2 - 2 dot or
  // -dot; the smaller value wins, the smaller index on equal values. x_t is recovered exactly from
  // the scaled operand.
  constexpr float kUnscale = L2 ? -0.5f : -1.0f;
  float be = __builtin_huge_valf();
  uint32_t bc = 0xFFFFFFFFu;
  int nband = 0;
  if (listed) {
#pragma unroll
    for (int i = 0; i < kAsgList - 1; ++i) nband += lg[i] <= band ? 1 : 0;
  }
  for (int i = 0; i < kAsgList - 1; ++i) {
    if (nband < 2 || i >= nband) break;
    const uint32_t c = lc[i];
    const f32x4* cr = reinterpret_cast<const f32x4*>(a.crow + static_cast<uint64_t>(c) * DP + h * H);
    float part = 0.0f;
    if (h == 0) {
#pragma unroll
      for (int s4 = 0; s4 < H / 4; ++s4) {
        const f32x4 cv = cr[s4];
#pragma unroll
        for (int e = 0; e < 4; ++e) part = part + (kUnscale * qreg[4 * s4 + e]) * cv[e];
      }
    }
    part = __shfl_xor(part, 32, 64);
    if (h == 1) {
#pragma unroll
      for (int s4 = 0; s4 < H / 4; ++s4) {
        const f32x4 cv = cr[s4];
#pragma unroll
        for (int e = 0; e < 4; ++e) part = part + (kUnscale * qreg[4 * s4 + e]) * cv[e];
      }
      const float ev = L2 ? a.aug[c] - 2.0f * part : -part;
      if (ev < be || (ev == be && c < bc)) {
        be = ev;
        bc = c;
      }
    }
  }
  if (!valid || h != 1) return;
  const bool decided = nband == 1 || (nband >= 2 && bc != 0xFFFFFFFFu);
  if (decided) {
    a.out32[p] = nband == 1 ? lc[0] : bc;
  } else {
    const uint32_t i = atomicAdd(&a.fb[0], 1u);
    a.fb[1 + i] = static_cast<uint32_t>(p);
  }
}

/// CentroidTable::nearest_batch for the points listed in list[1 .. list[0]] (those the MFMA pass
/// left open): a work-group per point, its threads across the centroids, each dot product summed
/// in order of t, then the smallest (value, index) among values below +inf (index 0 if none), as
/// the reference's "first strictly smaller" scan returns. Transposed centroids ct [dim][k].
constexpr int kListedCPT = 8;  // centroids per thread per pass
__global__ void __launch_bounds__(256) nearest_listed_kernel(NearestArgs a) {
  __shared__ float s_x[kAsgMaxDp];
  __shared__ uint64_t s_min[4];
  const int tid = threadIdx.x;
  const uint32_t cnt = a.list[0];
  for (uint32_t i = blockIdx.x; i < cnt; i += gridDim.x) {
    const uint64_t p = a.list[1 + i];
    __syncthreads();
    if (static_cast<uint32_t>(tid) < a.dim) s_x[tid] = a.x[p * a.x_stride + tid];
    __syncthreads();
    uint64_t best = ~0ull;
    for (uint32_t c0 = 0; c0 < a.k; c0 += 256 * kListedCPT) {
      float acc[kListedCPT];
#pragma unroll
      for (int e = 0; e < kListedCPT; ++e) acc[e] = 0.0f;
      for (uint32_t t = 0; t < a.dim; ++t) {
        const float xv = s_x[t];
#pragma unroll
        for (int e = 0; e < kListedCPT; ++e) {
          const uint32_t c = c0 + e * 256 + tid;
          const float cv = c < a.k ? a.ct[static_cast<uint64_t>(t) * a.k + c] : 0.0f;
          acc[e] = acc[e] + xv * cv;
        }
      }
#pragma unroll
      for (int e = 0; e < kListedCPT; ++e) {
        const uint32_t c = c0 + e * 256 + tid;
        const float d = a.max_ip ? -acc[e] : a.norms[c < a.k ? c : 0] - 2.0f * acc[e];
        if (c < a.k && d < __builtin_huge_valf()) {
          const uint64_t key = make_key(d, c);
          best = key < best ? key : best;
        }
      }
    }
    best = wave_min_u64(best);
    if ((tid & 63) == 0) s_min[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
      const uint64_t b = min(min(s_min[0], s_min[1]), min(s_min[2], s_min[3]));
      a.out32[p] = b == ~0ull ? 0u : static_cast<uint32_t>(b);
    }
  }
}

/// The MFMA assignment's centroid operand: rows [kp][dp] zero-padded, the augmented column and
/// (block 0, thread 0) the largest ||c||.
__global__ void assign_rows_kernel(const float* __restrict__ cent, const float* __restrict__ norms, uint32_t k,
                                   uint32_t dim, uint32_t dp, uint32_t kp, int max_ip, float* __restrict__ crow,
                                   float* __restrict__ aug) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<uint64_t>(kp) * dp) return;
  const uint32_t c = static_cast<uint32_t>(i / dp), t = static_cast<uint32_t>(i % dp);
  crow[i] = c < k && t < dim ? cent[static_cast<uint64_t>(c) * dim + t] : 0.0f;
  if (t == 0) aug[c] = c < k ? (max_ip ? 0.0f : norms[c]) : __builtin_huge_valf();
}

__global__ void __launch_bounds__(256) norm_max_kernel(const float* __restrict__ norms, uint32_t k,
                                                       float* __restrict__ rmax) {
  __shared__ float s_m[256];
  float m = 0.0f;
  for (uint32_t c = threadIdx.x; c < k; c += 256) m = fmaxf(m, norms[c]);
  s_m[threadIdx.x] = m;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) s_m[threadIdx.x] = fmaxf(s_m[threadIdx.x], s_m[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) rmax[0] = sqrtf(s_m[0]);
}

__global__ void assign_reset_kernel(uint32_t* fb) { fb[0] = 0; }

/// ||c||^2 summed in order (centroid_table.h:50-57) and the transposed table t[j][c].
__global__ void centroid_prep_kernel(const float* __restrict__ cent, uint32_t k, uint32_t dim,
                                     float* __restrict__ ct, float* __restrict__ norms) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= k) return;
  float norm = 0.0f;
  for (uint32_t j = 0; j < dim; ++j) {
    const float v = cent[static_cast<uint64_t>(c) * dim + j];
    ct[static_cast<uint64_t>(j) * k + c] = v;
    norm = norm + v * v;
  }
  if (norms) norms[c] = norm;
}

/// Codebook [m][256][dsub] -> per sub-space transposed [m][dsub][256].
__global__ void codebook_prep_kernel(const float* __restrict__ cb, uint32_t m, uint32_t dsub,
                                     float* __restrict__ cbt) {
  const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<uint64_t>(m) * 256 * dsub) return;
  const uint32_t t = e % dsub, c = (e / dsub) % 256, j = static_cast<uint32_t>(e / (256ull * dsub));
  cbt[(static_cast<uint64_t>(j) * dsub + t) * 256 + c] = cb[e];
}

/// Codebook [m][256][dsub] -> c-major [256][m][dsub] (the per-query table of the bank-rotated scan
/// is built from it with coalesced reads).
__global__ void codebook_cmajor_kernel(const float* __restrict__ cb, uint32_t m, uint32_t dsub,
                                       float* __restrict__ cbc) {
  const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<uint64_t>(m) * 256 * dsub) return;
  const uint32_t t = e % dsub, c = (e / dsub) % 256, j = static_cast<uint32_t>(e / (256ull * dsub));
  cbc[(static_cast<uint64_t>(c) * m + j) * dsub + t] = cb[e];
}

/// residual[p] = x[p] - centroid[assign[p]] (src/ivfpq_index.cc:243).
__global__ void residual_kernel(const float* __restrict__ x, const uint32_t* __restrict__ assign,
                                const float* __restrict__ cent, uint64_t n, uint32_t dim,
                                float* __restrict__ res) {
  const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n * dim) return;
  const uint64_t p = e / dim;
  const uint32_t j = static_cast<uint32_t>(e % dim);
  res[e] = x[e] - cent[static_cast<uint64_t>(assign[p]) * dim + j];
}

/// Impl::precompute (src/ivfpq_index.cc:117-127): sum_t r_t*r_t + (2*cl_t)*r_t, in order of t.
__global__ void precompute_kernel(const float* __restrict__ cent, const float* __restrict__ cb,
                                  uint32_t nlist, uint32_t dim, uint32_t m, float* __restrict__ pre) {
  const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<uint64_t>(nlist) * m * 256) return;
  const uint32_t dsub = dim / m;
  const uint32_t c = e % 256, j = (e / 256) % m;
  const uint64_t l = e / (256ull * m);
  const float* cl = cent + l * dim + static_cast<uint64_t>(j) * dsub;
  const float* r = cb + (static_cast<uint64_t>(j) * 256 + c) * dsub;
  float v = 0.0f;
  for (uint32_t t = 0; t < dsub; ++t) v = v + (r[t] * r[t] + 2.0f * cl[t] * r[t]);
  pre[e] = v;
}

/// pmax[l] = sum_j max_c |pre[l][j][c]|, summed in double and rounded up: with |score_l| and the
/// query's table bound, it bounds the magnitudes of every term of an L2 ADC sum over list l. One
/// block per list, one thread per sub-space.
__global__ void __launch_bounds__(256) pre_bound_kernel(const float* __restrict__ pre, uint32_t m,
                                                        float* __restrict__ pmax) {
  __shared__ double part[256];
  const uint32_t l = blockIdx.x;
  double mx = 0.0;
  for (uint32_t j = threadIdx.x; j < m; j += 256) {
    const float* row = pre + (static_cast<uint64_t>(l) * m + j) * 256;
    float r = 0.0f;
    for (uint32_t c = 0; c < 256; ++c) r = fmaxf(r, fabsf(row[c]));
    mx += static_cast<double>(r);
  }
  part[threadIdx.x] = mx;
  __syncthreads();
  for (uint32_t w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double v = part[0] * (1.0 + 1e-12);
    const float f = static_cast<float>(v);
    pmax[l] = static_cast<double>(f) < v ? __uint_as_float(__float_as_uint(f) + 1u) : f;
  }
}

/// term1[p] = sum_j pre[assign[p]][j][code_j], accumulated in double and rounded once.
__global__ void term1_kernel(const uint8_t* __restrict__ codes, uint32_t mp, const uint32_t* __restrict__ assign,
                             const float* __restrict__ pre, uint32_t m, uint64_t n, float* __restrict__ out) {
  const uint64_t p = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const float* pl = pre + static_cast<uint64_t>(assign[p]) * m * 256;
  const uint8_t* c = codes + p * mp;
  double s = 0.0;
  for (uint32_t j = 0; j < m; ++j) s += static_cast<double>(pl[j * 256 + c[j]]);
  out[p] = static_cast<float>(s);
}

/// The list of every CSR position (for term1 of lists installed as a whole).
__global__ void position_lists_kernel(const uint64_t* __restrict__ off, uint32_t nlist, uint64_t count,
                                      uint32_t* __restrict__ out) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count) return;
  uint32_t lo = 0, hi = nlist;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (off[mid] <= i) lo = mid; else hi = mid;
  }
  out[i] = lo;
}

/// Codes of n points from [n][m] (sub-space minor) to the padded CSR stride.
__global__ void pad_codes_kernel(const uint8_t* __restrict__ src, uint32_t m, uint32_t mp, uint64_t n,
                                 uint8_t* __restrict__ dst) {
  const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n * mp) return;
  const uint64_t p = e / mp;
  const uint32_t j = static_cast<uint32_t>(e % mp);
  dst[e] = j < m ? src[p * m + j] : 0;
}

/// New CSR from the old one plus a batch: old entry at old position i of list l moves by
/// shift[l]; batch entry b goes to dest[b].
struct ScatterArgs {
  const uint64_t* old_off;  // [nlist+1]
  const uint64_t* shift;    // [nlist] cumulative batch sizes of the lists before l
  uint32_t nlist;
  uint64_t old_count, n_new;
  const uint64_t* dest;     // [n_new]
  uint32_t mp, dim;
  const uint8_t* old_codes; const uint8_t* new_codes; uint8_t* codes;
  const float* old_t1; const float* new_t1; float* t1;
  const float* old_vec; const float* new_vec; float* vec;
};

__device__ __forceinline__ uint32_t list_of(const uint64_t* off, uint32_t nlist, uint64_t pos) {
  // last l with off[l] <= pos (lists may be empty)
  uint32_t lo = 0, hi = nlist;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (off[mid] <= pos) lo = mid; else hi = mid;
  }
  return lo;
}

__global__ void scatter_old_kernel(ScatterArgs a) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= a.old_count) return;
  const uint32_t l = list_of(a.old_off, a.nlist, i);
  const uint64_t dst = i + a.shift[l];
  for (uint32_t b = 0; b < a.mp; ++b) a.codes[dst * a.mp + b] = a.old_codes[i * a.mp + b];
  if (a.t1) a.t1[dst] = a.old_t1[i];
  if (a.vec) {
    for (uint32_t j = 0; j < a.dim; ++j) a.vec[dst * a.dim + j] = a.old_vec[i * a.dim + j];
  }
}

__global__ void scatter_new_kernel(ScatterArgs a) {
  const uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= a.n_new) return;
  const uint64_t dst = a.dest[b];
  for (uint32_t x = 0; x < a.mp; ++x) a.codes[dst * a.mp + x] = a.new_codes[b * a.mp + x];
  if (a.t1) a.t1[dst] = a.new_t1[b];
  if (a.vec) {
    for (uint32_t j = 0; j < a.dim; ++j) a.vec[dst * a.dim + j] = a.new_vec[b * a.dim + j];
  }
}

// ---- search: coarse scores and probe selection ------------------------------------------------

constexpr int kCoarseQ = 8;              // queries per coarse workgroup
constexpr uint64_t kCoarseSingleMaxQ = 128;  // smaller batches: one query per workgroup

/// Coarse scores (src/ivfpq_index.cc:285-297): L2: sum_j (q_j - c_j)^2; IP/cosine: -sum_j q_j c_j,
/// both in order of j (centroid_table.h:65-85). Stored as the reference's probe key. One thread
/// per centroid and QB queries per work-group (kCoarseQ, or 1 for small batches, which would
/// otherwise leave most CUs idle and compute padding queries); the query values are
/// block-uniform, so they come in through scalar loads and the vector unit does only the
/// arithmetic.
template <bool IP, int QB>
__global__ void __launch_bounds__(256) coarse_kernel(const float* __restrict__ Q, uint32_t nq, uint32_t dim,
                                                     const float* __restrict__ ct, uint32_t nlist,
                                                     float* __restrict__ scores) {
  constexpr int kCoarseQ = QB;
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  const uint32_t q0 = blockIdx.y * kCoarseQ;
  const uint32_t nb = min(static_cast<uint32_t>(kCoarseQ), nq - q0);
  const float* qrow[kCoarseQ];
#pragma unroll
  for (int b = 0; b < kCoarseQ; ++b) qrow[b] = Q + static_cast<uint64_t>(q0 + (b < static_cast<int>(nb) ? b : 0)) * dim;
  const uint32_t cc = c < nlist ? c : nlist - 1;
  float acc[kCoarseQ];
#pragma unroll
  for (int b = 0; b < kCoarseQ; ++b) acc[b] = 0.0f;
  // Centroid values are fetched JB at a time: with one query the sum chain is short, so more of
  // them must be in flight to cover the load latency (eight queries: 8 rather than 4 took the
  // select stage of 10k queries from 217 to 212 us).
  constexpr int JB = QB == 1 ? 16 : 8;
  uint32_t j = 0;
  for (; j + JB <= dim; j += JB) {
    float cj[JB];
#pragma unroll
    for (int t = 0; t < JB; ++t) cj[t] = ct[static_cast<uint64_t>(j + t) * nlist + cc];
#pragma unroll
    for (int b = 0; b < kCoarseQ; ++b) {
#pragma unroll
      for (int t = 0; t < JB; ++t) {
        const float qv = qrow[b][j + t];
        if (IP) {
          acc[b] = acc[b] + qv * cj[t];
        } else {
          const float d = qv - cj[t];
          acc[b] = acc[b] + d * d;
        }
      }
    }
  }
  for (; j < dim; ++j) {
    const float cj = ct[static_cast<uint64_t>(j) * nlist + cc];
#pragma unroll
    for (int b = 0; b < kCoarseQ; ++b) {
      const float qv = qrow[b][j];
      if (IP) {
        acc[b] = acc[b] + qv * cj;
      } else {
        const float d = qv - cj;
        acc[b] = acc[b] + d * d;
      }
    }
  }
  if (c >= nlist) return;
  for (uint32_t b = 0; b < nb; ++b) scores[static_cast<uint64_t>(q0 + b) * nlist + c] = IP ? -acc[b] : acc[b];
}

/// The nprobe smallest (score, list) per query, ascending (std::partial_sort of
/// src/ivfpq_index.cc:298-300, with ties broken by the list id). One wave per query. With up to
/// 64 * PER lists, every lane keeps its PER keys in registers; each step takes the wave minimum
/// of the lanes' current smallest keys, and the lane that supplied it moves to its next smallest.
template <int PER>
__global__ void __launch_bounds__(256) probe_select_kernel(const float* __restrict__ scores, uint32_t nq,
                                                           uint32_t nlist, uint32_t nprobe,
                                                           uint32_t* __restrict__ probes,
                                                           uint32_t* __restrict__ min_probe) {
  const int lane = threadIdx.x & 63;
  const uint32_t q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= nq) return;
  const float* sq = scores + static_cast<uint64_t>(q) * nlist;
  uint64_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t l = lane + 64 * i;
    float s = l < nlist ? sq[l] : 0.0f;
    s = s == s ? s : __builtin_huge_valf();
    key[i] = l < nlist ? make_key(s, l) : ~0ull;
  }
  auto smallest = [&]() {
    uint64_t b = key[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) b = key[i] < b ? key[i] : b;
    return b;
  };
  uint64_t cur = smallest();
  if (nprobe <= 64) {
    // Threshold T = the nprobe-th smallest of the 64 lane minima (nprobe <= 32), or of the lanes'
    // two smallest keys each (33..64: the lane minima alone admit a few hundred keys there): at
    // least nprobe distinct keys are <= T, so the nprobe smallest keys are all <= T. The keys <= T
    // (usually a few dozen past nprobe) are sorted in LDS; more than 128 of them falls through to
    // the selection loop below.
    uint64_t T;
    if (nprobe <= 32) {
      uint64_t v = cur;
#pragma unroll
      for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          const uint64_t o = lane_xor_u64(v, stride);
          const bool keep_min = ((lane & stride) == 0) == ((lane & size) == 0);
          v = keep_min ? (o < v ? o : v) : (o > v ? o : v);
        }
      }
      T = __shfl(v, static_cast<int>(nprobe) - 1, 64);
    } else {
      uint64_t second = ~0ull;
#pragma unroll
      for (int i = 0; i < PER; ++i) second = key[i] != cur && key[i] < second ? key[i] : second;
      uint64_t two[2] = {cur, second};
      wave_sort<2>(two);  // element e = i * 64 + lane in two[i]
      const int e = static_cast<int>(nprobe) - 1;
      T = __shfl(e < 64 ? two[0] : two[1], e & 63, 64);
    }
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) n += static_cast<uint32_t>(__popcll(__ballot(key[i] <= T)));
    if (n <= 128) {
      __shared__ uint64_t s_cand[4][128];
      uint64_t* cand = s_cand[threadIdx.x >> 6];
      uint32_t at = 0;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const bool pass = key[i] <= T;
        const uint64_t mk = __ballot(pass);
        if (pass) cand[at + lane_rank(mk)] = key[i];
        at += static_cast<uint32_t>(__popcll(mk));
      }
      for (uint32_t e = at + lane; e < 128; e += 64) cand[e] = ~0ull;
      __builtin_amdgcn_wave_barrier();
      uint64_t x[2] = {cand[lane], cand[lane + 64]};
#pragma unroll
      for (int size = 2; size <= 128; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          if (stride == 64) {
            const uint64_t lo = x[0] < x[1] ? x[0] : x[1], hi = x[0] < x[1] ? x[1] : x[0];
            x[0] = lo;
            x[1] = hi;
          } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int e = lane + 64 * h;
              const uint64_t o = lane_xor_u64(x[h], stride);
              const bool keep_min = ((e & stride) == 0) == ((e & size) == 0);
              x[h] = keep_min ? (o < x[h] ? o : x[h]) : (o > x[h] ? o : x[h]);
            }
          }
        }
      }
      const uint32_t l = static_cast<uint32_t>(x[0]);
      if (static_cast<uint32_t>(lane) < nprobe) probes[static_cast<uint64_t>(q) * nprobe + lane] = l;
      if (min_probe) {
        uint32_t mn = static_cast<uint32_t>(lane) < nprobe ? l : 0xFFFFFFFFu;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mn = min(mn, static_cast<uint32_t>(__shfl_xor(mn, off, 64)));
        if (lane == 0) min_probe[q] = mn;
      }
      return;
    }
  }
  uint32_t mn = 0xFFFFFFFFu;
  for (uint32_t p = 0; p < nprobe; ++p) {
    const uint64_t best = wave_min_u64(cur);
    if (lane == 0) probes[static_cast<uint64_t>(q) * nprobe + p] = static_cast<uint32_t>(best);
    mn = min(mn, static_cast<uint32_t>(best));
    if (cur == best) {
#pragma unroll
      for (int i = 0; i < PER; ++i) key[i] = key[i] == best ? ~0ull : key[i];
      cur = smallest();
    }
  }
  if (min_probe && lane == 0) min_probe[q] = mn;
}

/// Same selection for any nlist: a lane rescans its strided share above the last key popped.
__global__ void __launch_bounds__(256) probe_select_any_kernel(const float* __restrict__ scores, uint32_t nq,
                                                               uint32_t nlist, uint32_t nprobe,
                                                               uint32_t* __restrict__ probes,
                                                               uint32_t* __restrict__ min_probe) {
  const int lane = threadIdx.x & 63;
  const uint32_t q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= nq) return;
  const float* sq = scores + static_cast<uint64_t>(q) * nlist;
  auto my_next = [&](uint64_t above, bool first) {
    uint64_t best = ~0ull;
    for (uint32_t l = lane; l < nlist; l += 64) {
      float s = sq[l];
      s = s == s ? s : __builtin_huge_valf();
      const uint64_t key = make_key(s, l);
      if ((first || key > above) && key < best) best = key;
    }
    return best;
  };
  uint64_t cur = my_next(0, true);
  uint32_t mn = 0xFFFFFFFFu;
  for (uint32_t p = 0; p < nprobe; ++p) {
    const uint64_t best = wave_min_u64(cur);
    if (lane == 0) probes[static_cast<uint64_t>(q) * nprobe + p] = static_cast<uint32_t>(best);
    mn = min(mn, static_cast<uint32_t>(best));
    if (cur == best) cur = my_next(best, false);
  }
  if (min_probe && lane == 0) min_probe[q] = mn;
}

// ---- search: coarse scores on the matrix unit ----------------------------------------------------
//
// Batches of at least kCgMinQueries queries (kCgMinQueriesWide above 32 probes) score the
// centroids on the matrix unit: g_c =
// ||c||^2 - 2<q,c> for L2 (the query enters scaled by -2, exact, and one more MFMA step adds the
// augmented column ||c||^2 of the assignment operand) or -<q,c> for inner product and cosine. g
// differs from the reference's in-order sum e_c (src/internal/centroid_table.h:65-85) by the
// constant ||q||^2 (L2) and by rounding: |(||q||^2 + g_c) - e_c| <= delta with the assignment
// kernel's bound, delta = (4 (dp + 1) + 16) u (P + R)^2 for L2 and (4 (dp + 1) + 16) u P R for the
// inner product (P = ||q||, R = the largest ||c||). Let G_n be the nprobe-th smallest g. The
// nprobe lists of smallest g all have e <= G_n + ||q||^2 + delta, so the nprobe-th smallest e is at
// most that, and every list of the reference's probe set has g <= G_n + 2 delta. Those lists (the
// band) are re-scored in the reference's order and arithmetic and the nprobe smallest (e, list)
// are the probes, exactly as the in-order kernels would choose them. The exact scores of the band
// overwrite their approximate values in the score array, which the scan then reads for the probed
// lists only.

constexpr int kCgWaves = 8;               // 4 x 2 over the work-group's output tile
constexpr int kCgThreads = kCgWaves * 64;
constexpr uint32_t kCgTileQ = 128;        // queries per work-group tile (32 per wave row)
constexpr uint32_t kCgTileC = 128;        // centroids per work-group tile (64 per wave column)
constexpr uint32_t kCgKC = 32;            // dims per LDS chunk
constexpr int kCgPitch = kCgKC + 4;       // LDS row pitch in floats: conflict-free 16-byte reads
constexpr int kCgOutPitch = 64 + 4;       // the epilogue's per-wave block of 32 queries x 64 centroids
// Smallest batches scored on the matrix unit (smaller ones: coarse_kernel); the matrix path costs a
// nearly fixed 34-39 us at nprobe <= 32 and 45 us at 64, the in-order kernel grows with the batch
// (1M x 128, 2048 lists, select stage: 200 queries 42.4 -> 34.4 us, 1,000 queries 52.5 -> 35.1 us
// at nprobe 8; 100 queries 35.9 vs 38.6 us at nprobe 32; 300 queries 44.6 vs 45.3 us at nprobe 64).
constexpr uint64_t kCgMinQueries = 192;
constexpr uint64_t kCgMinQueriesWide = 512;  // nprobe above 32
constexpr uint32_t kCgMaxProbes = 64;
constexpr uint32_t kCgMaxLists = 64 * 32;
constexpr int kBandCap = 128;             // band members re-scored and sorted in registers
constexpr uint32_t kBandKC = 16;          // dims per staged chunk of the band's centroid rows
constexpr int kBandPitch = kBandKC + 4;   // staged row pitch in floats
static_assert(kCgWaves * 32 * kCgOutPitch <= 2 * static_cast<int>(kCgTileQ + kCgTileC) * kCgPitch,
              "the epilogue blocks fit the operand buffers");

struct CoarseGemmArgs {
  const float* Q;         // [nq][dim], 16-byte aligned rows, dim a multiple of 4
  uint32_t nq, dim;
  const float* crow;      // [kp][dp] centroid rows, zero padded (the assignment operand)
  const float* aug;       // [kp] ||c||^2; read for L2 only
  uint32_t kp, dp, nlist;
  uint32_t ncb;           // centroid tiles
  uint32_t qb_per_xcd;    // query tiles per XCD
  uint32_t nqb;           // query tiles
  float* g;               // [nq][nlist] approximate scores
};

/// g for one 128-query x 128-centroid tile per work-group: wave w owns queries 32 (w % 4) .. and
/// centroids 64 (w / 4) .. of the tile (two 32 x 32 MFMA blocks sharing the query operand). Both
/// operands pass through LDS in chunks of 32 dims, double buffered, the next chunk's global loads
/// in flight during this chunk's MFMAs. Each wave's finished block goes through LDS so that the
/// scores leave as whole 256-byte row segments. Work-group b runs on XCD b % 8 (the dispatcher's
/// round robin); each XCD takes a contiguous range of query tiles with all their centroid tiles,
/// so its L2 holds its queries and the whole centroid operand.
template <bool L2>
__global__ void __launch_bounds__(kCgThreads) coarse_gemm_kernel(CoarseGemmArgs a) {
  __shared__ __attribute__((aligned(16))) float s_buf[2 * (kCgTileC + kCgTileQ) * kCgPitch];
  auto s_c = [&](int buf) { return s_buf + buf * kCgTileC * kCgPitch; };
  auto s_qt = [&](int buf) { return s_buf + 2 * kCgTileC * kCgPitch + buf * kCgTileQ * kCgPitch; };
  const uint32_t r = blockIdx.x >> 3;
  const uint32_t qb = (blockIdx.x & 7u) * a.qb_per_xcd + r / a.ncb;
  const uint32_t cb = r % a.ncb;
  if (qb >= a.nqb) return;  // whole work-group
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const uint32_t wq = wave & 3, wc = wave >> 2;
  const uint32_t q0 = qb * kCgTileQ, c0 = cb * kCgTileC;
  constexpr float kScale = L2 ? -2.0f : -1.0f;

  // Chunk element e = tid + 512 i: row e / 8, dims 4 (e % 8) .. of the chunk. The loads are
  // unconditional (clamped addresses) and nothing uses their values before the store to LDS, so
  // they stay in flight across the chunk's MFMAs; rows past the batch and dims past the query's
  // width become zeros (and the scaling is applied) only at the store.
  f32x4 st_c[2], st_q[2];
  auto load_chunk = [&](uint32_t kc) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t e = static_cast<uint32_t>(tid) + kCgThreads * i;
      const uint32_t row = e >> 3, d = kc + 4 * (e & 7u);
      const uint32_t c = min(c0 + row, a.kp - 1);
      st_c[i] = *reinterpret_cast<const f32x4*>(a.crow + static_cast<uint64_t>(c) * a.dp + d);
      const uint32_t p = min(q0 + row, a.nq - 1);
      st_q[i] = *reinterpret_cast<const f32x4*>(a.Q + static_cast<uint64_t>(p) * a.dim + min(d, a.dim - 4));
    }
  };
  auto store_chunk = [&](int buf, uint32_t kc) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t e = static_cast<uint32_t>(tid) + kCgThreads * i;
      const uint32_t row = e >> 3, d = kc + 4 * (e & 7u);
      const uint32_t o = row * kCgPitch + 4 * (e & 7u);
      const float sq = q0 + row < a.nq && d < a.dim ? kScale : 0.0f;
      *reinterpret_cast<f32x4*>(&s_c(buf)[o]) = st_c[i];
      *reinterpret_cast<f32x4*>(&s_qt(buf)[o]) = f32x4{sq * st_q[i][0], sq * st_q[i][1], sq * st_q[i][2], sq * st_q[i][3]};
    }
  };

  f32x16 acc[2] = {};  // the wave's two centroid blocks
  const uint32_t nk = a.dp / kCgKC;
  load_chunk(0);
  store_chunk(0, 0);
  __syncthreads();
  for (uint32_t kc = 0; kc < nk; ++kc) {
    const int buf = kc & 1;
    const bool more = kc + 1 < nk;
    if (more) load_chunk((kc + 1) * kCgKC);
    // Lane (j, h) feeds k = h: dims [16 h, 16 h + 16) of the chunk, four per 16-byte read.
    const float* pc = s_c(buf) + (64 * wc + j) * kCgPitch + 16 * h;
    const float* pq = s_qt(buf) + (32 * wq + j) * kCgPitch + 16 * h;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const f32x4 c0v = *reinterpret_cast<const f32x4*>(pc + 4 * s4);
      const f32x4 c1v = *reinterpret_cast<const f32x4*>(pc + 32 * kCgPitch + 4 * s4);
      const f32x4 qv = *reinterpret_cast<const f32x4*>(pq + 4 * s4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(c0v[e], qv[e], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(c1v[e], qv[e], acc[1], 0, 0, 0);
      }
    }
    if (more) store_chunk(buf ^ 1, (kc + 1) * kCgKC);
    __syncthreads();
  }
  if (L2) {
    // (||c||^2, 0) . (1, 0): lane half 0 feeds the norm and the one.
    const float qaug = h == 0 ? 1.0f : 0.0f;
#pragma unroll
    for (int bc = 0; bc < 2; ++bc) {
      const uint32_t c = min(c0 + 64 * wc + 32 * bc + j, a.kp - 1);
      const float ca = h == 0 ? a.aug[c] : 0.0f;
      acc[bc] = __builtin_amdgcn_mfma_f32_32x32x2f32(ca, qaug, acc[bc], 0, 0, 0);
    }
  }
  // D[row][col]: col = query j, row = centroid 8 (r / 4) + 4 h + r % 4 of the block in register r.
  // The wave's block goes to LDS as 32 query rows of 64 centroids (the operand buffers are free
  // after the loop's last barrier), then out in 256-byte row segments.
  float* so = s_buf + wave * 32 * kCgOutPitch;
#pragma unroll
  for (int bc = 0; bc < 2; ++bc) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      *reinterpret_cast<f32x4*>(&so[j * kCgOutPitch + 32 * bc + 8 * r4 + 4 * h]) =
          f32x4{acc[bc][4 * r4], acc[bc][4 * r4 + 1], acc[bc][4 * r4 + 2], acc[bc][4 * r4 + 3]};
    }
  }
  __builtin_amdgcn_wave_barrier();
  const bool vec_out = (a.nlist & 3u) == 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 4 * i + (lane >> 4), col = 4 * (lane & 15);
    const uint32_t p = q0 + 32 * wq + row;
    const uint32_t c = c0 + 64 * wc + col;
    if (p >= a.nq) continue;
    const f32x4 v = *reinterpret_cast<const f32x4*>(&so[row * kCgOutPitch + col]);
    float* dst = a.g + static_cast<uint64_t>(p) * a.nlist + c;
    if (vec_out) {
      if (c < a.nlist) *reinterpret_cast<f32x4*>(dst) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (c + e < a.nlist) dst[e] = v[e];
      }
    }
  }
}

/// The L2 ranking's rounding bound for one query (one wave; every lane returns it): (2m + 16) u
/// times (the largest |score_l| + pmax[l] over the probed lists, of which each lane brings its
/// share in bp, plus T_q = 2 sum_j ||q_j|| cmax[j]), rounded up. See adc_bound_kernel.
__device__ float adc_delta(const float* qv, uint32_t m, uint32_t dsub, const float* __restrict__ cmax, float bp) {
  const int lane = threadIdx.x & 63;
  double tsum = 0.0;
  for (uint32_t j = lane; j < m; j += 64) {
    double norm2 = 0.0;
    for (uint32_t t = 0; t < dsub; ++t) {
      const double v = qv[static_cast<uint64_t>(j) * dsub + t];
      norm2 += v * v;
    }
    tsum += sqrt(norm2) * static_cast<double>(cmax[j]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) tsum += __shfl_xor(tsum, off, 64);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) bp = fmaxf(bp, __shfl_xor(bp, off, 64));
  // (1 + 2^-20) covers the float rounding of |score| + pmax, the double sums and dsub u; a NaN or
  // overflowing bound stays non-finite and certifies nothing.
  const double tq = 2.0 * tsum;
  const double d = (2.0 * m + 16.0) / 16777216.0 * ((static_cast<double>(bp) + tq) * (1.0 + 1.0 / 1048576.0));
  const float df = static_cast<float>(d);
  return static_cast<double>(df) < d ? __uint_as_float(__float_as_uint(df) + 1u) : df;
}

struct BandArgs {
  const float* Q;          // [nq][dim], 16-byte aligned rows, dim a multiple of 4, at most kAsgMaxDp
  uint32_t nq, dim;
  const float* cent;       // [nlist][dim]
  uint32_t nlist, nprobe;  // nprobe <= kCgMaxProbes
  const float* rmax;       // [1] the largest ||c||
  float coef;              // (4 (dp + 1) + 16) * 2^-24
  float* scores;           // [nq][nlist]: approximate g in; the exact score of every re-scored list out
  uint32_t* probes;        // [nq][nprobe]
  uint32_t* min_probe;     // [nq] smallest probed list, or null
  // L2 with the precomputed table: the scan's certificate bound per query (adc_delta), or null.
  float* adc_bound;        // [nq]
  const float* cmax;       // [m]
  const float* pmax;       // [nlist]
  uint32_t m, dsub;
  uint32_t* fb_count;      // the scan's count of uncertified queries, reset here (with adc_bound)
};

/// The reference's coarse score of list l: sum_j (q_j - c_j)^2 or -sum_j q_j c_j in order of j,
/// unfused (src/internal/centroid_table.h:65-85), the query from LDS.
template <bool IP>
__device__ __forceinline__ float coarse_exact(const float* __restrict__ sq, const float* __restrict__ crow,
                                              uint32_t dim) {
  float acc = 0.0f;
  for (uint32_t j = 0; j < dim; j += 4) {
    const f32x4 c = *reinterpret_cast<const f32x4*>(crow + j);
    const f32x4 q = *reinterpret_cast<const f32x4*>(sq + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (IP) {
        acc = acc + q[e] * c[e];
      } else {
        const float d = q[e] - c[e];
        acc = acc + d * d;
      }
    }
  }
  return IP ? -acc : acc;
}

/// coarse_exact as a call: the every-list path of the band kernel runs it 32 times per lane.
template <bool IP>
__device__ __attribute__((noinline)) float coarse_exact_call(const float* sq, const float* crow, uint32_t dim) {
  return coarse_exact<IP>(sq, crow, dim);
}

/// The probes of one query per wave from the approximate scores (std::partial_sort of
/// src/ivfpq_index.cc:298-300, ties broken by the list id). U, the nprobe-th smallest of the lanes'
/// minima (nprobe <= 32) or of their two smallest scores each (33..64), has at least nprobe scores
/// at or below it, so U >= G_n and every list with g <= U + 2 delta is re-scored exactly: a
/// superset of the band, usually a few lists past nprobe. When that set exceeds kBandCap, G_n
/// itself is found (bit by bit) and the band proper is re-scored; a band beyond kBandCap (many
/// lists within rounding of each other) re-scores every list of the query.
/// Lane `lane` holds lists 256 i + 4 lane + e in og[4 i + e] (the scores as ordered 32-bit keys;
/// a non-finite approximation comes with a non-finite delta, which admits every list).
template <bool IP, int PER4>
__global__ void __launch_bounds__(256) coarse_band_kernel(BandArgs a) {
  constexpr int PER = 4 * PER4;
  __shared__ __attribute__((aligned(16))) float s_q[4][kAsgMaxDp];
  __shared__ uint32_t s_u[4][kBandCap];
  __shared__ __attribute__((aligned(16))) float s_rows[4][64 * kBandPitch];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const uint32_t q = blockIdx.x * 4 + w;
  // The scan's count of uncertified queries starts at zero (the previous search's kernels, on the
  // same stream, are done with it).
  if (a.fb_count && blockIdx.x == 0 && threadIdx.x == 0) *a.fb_count = 0u;
  if (q >= a.nq) return;  // whole wave
  const uint32_t dim = a.dim, nlist = a.nlist, nprobe = a.nprobe;
  float pp = 0.0f;
  for (uint32_t d = 4 * lane; d < dim; d += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(a.Q + static_cast<uint64_t>(q) * dim + d);
    *reinterpret_cast<f32x4*>(&s_q[w][d]) = v;
    pp = pp + v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) pp = pp + __shfl_xor(pp, off, 64);
  // ||q|| from a sum in some order: its relative error is far inside the bound's factor of two.
  const float P = sqrtf(pp), R = a.rmax[0];
  const float delta = IP ? a.coef * P * R : a.coef * (P + R) * (P + R);
  // Ordered key of g + 2 delta rounded up: the next float above the float sum covers its rounding;
  // a non-finite limit admits everything.
  auto band_limit = [&](uint32_t gkey) {
    const float s = ordered_to_float(gkey) + 2.0f * delta;
    if (!(s < __builtin_huge_valf())) return 0xFFFFFFFFu;
    const float up = s == 0.0f ? __uint_as_float(1u)
                               : __uint_as_float(s > 0.0f ? __float_as_uint(s) + 1u : __float_as_uint(s) - 1u);
    return float_to_ordered(up);
  };

  float* sc = a.scores + static_cast<uint64_t>(q) * nlist;
  const bool vec = (nlist & 3u) == 0;
  uint32_t og[PER];
#pragma unroll
  for (int i = 0; i < PER4; ++i) {
    const uint32_t l0 = 256 * i + 4 * lane;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (vec && l0 < nlist) {
      v = *reinterpret_cast<const f32x4*>(sc + l0);
    } else if (!vec) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = l0 + e < nlist ? sc[l0 + e] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) og[4 * i + e] = l0 + e < nlist ? float_to_ordered(v[e]) : 0xFFFFFFFFu;
  }
  auto count_at_most = [&](uint32_t lim) {
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) n += static_cast<uint32_t>(__popcll(__ballot(og[i] <= lim)));
    return n;
  };
  uint32_t U;
  if (nprobe <= 32) {
    uint32_t m1 = og[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) m1 = min(m1, og[i]);
    uint32_t one[1] = {m1};
    wave_sort_u32<1>(one);
    U = static_cast<uint32_t>(__shfl(static_cast<int>(one[0]), static_cast<int>(nprobe) - 1, 64));
  } else {
    uint32_t m1 = 0xFFFFFFFFu, m2 = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t v = og[i];
      m2 = v < m1 ? m1 : min(v, m2);
      m1 = min(v, m1);
    }
    uint32_t two[2] = {m1, m2};
    wave_sort_u32<2>(two);
    const int e = static_cast<int>(nprobe) - 1;
    U = static_cast<uint32_t>(__shfl(static_cast<int>(e < 64 ? two[0] : two[1]), e & 63, 64));
  }
  // A saturated limit (non-finite bound) sends the query to the exact re-score of every list.
  uint32_t lim = band_limit(U);
  uint32_t n = lim == 0xFFFFFFFFu ? 0xFFFFFFFFu : count_at_most(lim);
  if (n > static_cast<uint32_t>(kBandCap) && lim != 0xFFFFFFFFu) {
    // U too loose: G_n bit by bit, the smallest t with at least nprobe scores at or below it.
    uint32_t gn = 0;
    for (int b = 31; b >= 0; --b) {
      const uint32_t probe = gn | ((1u << b) - 1u);
      if (count_at_most(probe) < nprobe) gn |= 1u << b;
    }
    lim = band_limit(gn);
    n = lim == 0xFFFFFFFFu ? 0xFFFFFFFFu : count_at_most(lim);
  }
  uint32_t* pr = a.probes + static_cast<uint64_t>(q) * nprobe;
  if (n <= static_cast<uint32_t>(kBandCap)) {
    uint32_t* su = s_u[w];
    {
      uint32_t at = 0;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const bool pass = og[i] <= lim;
        const uint64_t mk = __ballot(pass);
        if (pass) su[at + lane_rank(mk)] = 256 * (i / 4) + 4 * lane + (i % 4);
        at += static_cast<uint32_t>(__popcll(mk));
      }
      __builtin_amdgcn_wave_barrier();
    }
    // Exact scores, 64 lists at a time: 16-dim chunks of their centroid rows are staged in LDS
    // with coalesced loads (four lanes per row), then each lane sums its list's row in order.
    uint64_t key[2] = {~0ull, ~0ull};
    float* rows = s_rows[w];
    for (uint32_t base = 0; base < n; base += 64) {
      const uint32_t nbp = min(64u, n - base);
      const uint32_t myl = static_cast<uint32_t>(lane) < nbp ? su[base + lane] : 0u;
      const float* src[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t b = 16 * i + (lane >> 2);
        src[i] = a.cent + static_cast<uint64_t>(b < nbp ? su[base + b] : 0u) * dim + 4 * (lane & 3);
      }
      float acc = 0.0f;
      for (uint32_t dc = 0; dc < dim; dc += kBandKC) {
        const bool part_in = dc + 4 * (lane & 3) < dim;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t b = 16 * i + (lane >> 2);
          if (b < nbp && part_in) {
            *reinterpret_cast<f32x4*>(&rows[b * kBandPitch + 4 * (lane & 3)]) = *reinterpret_cast<const f32x4*>(src[i] + dc);
          }
        }
        __builtin_amdgcn_wave_barrier();
        if (static_cast<uint32_t>(lane) < nbp) {
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) {
            const uint32_t d = dc + 4 * s4;
            if (d < dim) {
              const f32x4 c = *reinterpret_cast<const f32x4*>(&rows[lane * kBandPitch + 4 * s4]);
              const f32x4 qv = *reinterpret_cast<const f32x4*>(&s_q[w][d]);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                if (IP) {
                  acc = acc + qv[e] * c[e];
                } else {
                  const float df = qv[e] - c[e];
                  acc = acc + df * df;
                }
              }
            }
          }
        }
        __builtin_amdgcn_wave_barrier();
      }
      if (static_cast<uint32_t>(lane) < nbp) {
        const float s = IP ? -acc : acc;
        sc[myl] = s;
        const uint64_t kk = make_key(s == s ? s : __builtin_huge_valf(), myl);
        if (base == 0) {
          key[0] = kk;
        } else {
          key[1] = kk;
        }
      }
    }
    if (n > 64) {
      wave_sort<2>(key);
    } else {
      uint64_t one[1] = {key[0]};
      wave_sort<1>(one);
      key[0] = one[0];
    }
    const uint32_t l = static_cast<uint32_t>(key[0]);
    const bool probed = static_cast<uint32_t>(lane) < nprobe;
    if (probed) pr[lane] = l;
    if (a.min_probe) {
      uint32_t mn = probed ? l : 0xFFFFFFFFu;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mn = min(mn, static_cast<uint32_t>(__shfl_xor(mn, off, 64)));
      if (lane == 0) a.min_probe[q] = mn;
    }
    if (a.adc_bound) {
      const float bp = probed ? fabsf(ordered_to_float(static_cast<uint32_t>(key[0] >> 32))) + a.pmax[l] : 0.0f;
      const float d = adc_delta(s_q[w], a.m, a.dsub, a.cmax, bp);
      if (lane == 0) a.adc_bound[q] = d;
    }
    return;
  }
  // Many lists within rounding of each other: every list's exact score, then the nprobe smallest
  // (score, list) one at a time.
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t l = 256 * (i / 4) + 4 * lane + (i % 4);
    og[i] = 0xFFFFFFFFu;
    if (l < nlist) {
      const float s = coarse_exact_call<IP>(s_q[w], a.cent + static_cast<uint64_t>(l) * dim, dim);
      sc[l] = s;
      og[i] = float_to_ordered(s == s ? s : __builtin_huge_valf());
    }
  }
  auto lane_best = [&]() {
    uint64_t b = ~0ull;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint64_t k = og[i] == 0xFFFFFFFFu ? ~0ull
                                              : (static_cast<uint64_t>(og[i]) << 32) | (256 * (i / 4) + 4 * lane + (i % 4));
      b = k < b ? k : b;
    }
    return b;
  };
  uint64_t cur = lane_best();
  uint32_t mn = 0xFFFFFFFFu;
  float bp = 0.0f;
  for (uint32_t p = 0; p < nprobe; ++p) {
    const uint64_t best = wave_min_u64(cur);
    const uint32_t bl = static_cast<uint32_t>(best);
    if (lane == 0) pr[p] = bl;
    mn = min(mn, bl);
    if (a.adc_bound && lane == 0) bp = fmaxf(bp, fabsf(ordered_to_float(static_cast<uint32_t>(best >> 32))) + a.pmax[bl]);
    if (cur == best) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if (256 * (i / 4) + 4 * lane + (i % 4) == bl) og[i] = 0xFFFFFFFFu;
      }
      cur = lane_best();
    }
  }
  if (a.min_probe && lane == 0) a.min_probe[q] = mn;
  if (a.adc_bound) {
    const float d = adc_delta(s_q[w], a.m, a.dsub, a.cmax, bp);
    if (lane == 0) a.adc_bound[q] = d;
  }
}

// ---- search: the scan ---------------------------------------------------------------------------

constexpr int kScanThreads = 256;
constexpr int kCandCap = 2048;       // LDS candidate buffer (u64 keys) for keep_sel <= kMaxKeepSel
constexpr int kScanRound = 4;        // codes per thread between buffer checks
constexpr uint32_t kMaxKeepSel = kCandCap - kScanThreads * kScanRound;  // 1024
// Larger m keeps the block-buffer scan's per-query table (m x 256 floats) in global memory.
constexpr uint32_t kScanMaxLdsM = 128;
constexpr size_t kScanMaxLds = 150 * 1024;  // dynamic LDS the block-buffer scan takes at most
constexpr uint64_t kScanGlobalTableBytes = 256ull << 20;  // bound on those tables, all work-groups
constexpr uint64_t kScanGlobalCandBytes = 512ull << 20;   // and on candidate buffers in global memory
// Larger selections take a larger buffer: keep_sel + kScanThreads * kScanRound slots, rounded up to
// a power of two, as far as LDS allows.

// Scan order of the queries. Queries whose probe sets overlap read the same lists; run next to each
// other, they find those lists in L2. Each query is keyed by the smallest list id it probes (a
// min-hash of its probe set: two queries share it with probability equal to the Jaccard
// similarity of their probe sets), and a counting sort over the keys gives the block -> query map.
// The order changes only which block scans which query, never a query's result.

/// order = the queries sorted by key (counting sort, LDS counts over the nlist keys; one block).
/// Within a key the order is whatever the LDS atomics give.
__global__ void __launch_bounds__(1024) probe_order_kernel(const uint32_t* __restrict__ key, uint32_t nq,
                                                           uint32_t nlist, uint32_t* __restrict__ order) {
  extern __shared__ uint32_t s_count[];  // [nlist]
  __shared__ uint32_t s_part[33];        // wave totals, wave bases, chunk total
  __shared__ uint32_t s_carry;
  const uint32_t tid = threadIdx.x;
  for (uint32_t g = tid; g < nlist; g += 1024) s_count[g] = 0u;
  if (tid == 0) s_carry = 0u;
  __syncthreads();
  for (uint32_t q = tid; q < nq; q += 1024) atomicAdd(&s_count[key[q]], 1u);
  __syncthreads();
  // Exclusive prefix sum over the counts, 1024 at a time: an inclusive scan inside each wave
  // (shuffles), the 16 wave totals scanned by wave 0, then every count offset by its wave's base.
  const uint32_t lane = tid & 63u, wave = tid >> 6;
  for (uint32_t b = 0; b < nlist; b += 1024) {
    const uint32_t v = b + tid < nlist ? s_count[b + tid] : 0u;
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off, 64);
      if (lane >= static_cast<uint32_t>(off)) incl += o;
    }
    if (lane == 63) s_part[wave] = incl;
    __syncthreads();
    if (wave == 0) {
      const uint32_t t = lane < 16 ? s_part[lane] : 0u;
      uint32_t ti = t;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const uint32_t o = __shfl_up(ti, off, 64);
        if (lane >= static_cast<uint32_t>(off)) ti += o;
      }
      if (lane < 16) s_part[16 + lane] = ti - t;  // exclusive base of wave `lane`
      if (lane == 15) s_part[32] = ti;            // the chunk's total
    }
    __syncthreads();
    if (b + tid < nlist) s_count[b + tid] = s_carry + s_part[16 + wave] + incl - v;
    __syncthreads();
    if (tid == 0) s_carry += s_part[32];
    __syncthreads();
  }
  for (uint32_t q = tid; q < nq; q += 1024) order[atomicAdd(&s_count[key[q]], 1u)] = q;
}

struct ScanArgs {
  uint32_t nq, k, m, mp, dsub, dim, nlist, nprobe;
  int mode;
  const float* Q;          // [nq][dim] prepared
  const float* scores;     // [nq][nlist] probe keys
  const uint32_t* probes;  // [nq][nprobe]
  const uint64_t* off;     // [nlist+1]
  const uint8_t* codes;    // [count][mp]
  const float* t1;         // [count] (mode pre)
  const float* pre;        // [nlist][m][256] (mode pre)
  const float* cbt;        // [m][dsub][256]
  const float* cbc;        // [256][m][dsub]
  const float* cent;       // [nlist][dim] (mode residual)
  const float* vec;        // [count][dim] or null
  const uint64_t* bitmap;  // admitted positions, or null
  uint32_t keep, keep_sel;
  uint32_t cand_cap;  // block-buffer scan: LDS candidate slots (a power of two, >= kCandCap)
  int refine;
  int exact_all;  // block-buffer scan: exact distances of every probed vector (saturated refine)
  uint64_t* out_refs;
  float* out_dist;
  const uint32_t* order;  // [nq] block -> query of the streaming scan, or null
  // Sliced queries of the streaming scan: blocks [0, nwhole) scan one query each; the rest scan
  // one of `parts` slices of a query's probed codes and leave their best keep keys in part_keys;
  // the slice that finishes last merges them (part_done counts finished slices, reset by the
  // merging block).
  uint32_t nwhole, parts;
  uint64_t* part_keys;  // [nq - nwhole][parts][keep]
  uint32_t* part_cnt;   // [nq - nwhole][parts]; bit 31 set: that slice's selection is uncertified
  uint32_t* part_done;  // [nq - nwhole], zero between searches
  // Mode pre: the approximate ranking's certificate (adc_bound_kernel) and the queries it could not
  // certify, which the block-buffer scan then recomputes with exact sums (exact_pre).
  const float* delta;   // [nq]
  uint32_t* fallback;   // [nq]
  uint32_t* nfallback;
  int exact_pre;        // block-buffer scan: the reference's sum for every code, no re-score
  const uint32_t* qlist;   // block-buffer scan over listed queries (block b runs qlist[b] while
  const uint32_t* qcount;  // b < *qcount), or null: block b runs query b
  // Block-buffer scan with m above kScanMaxLdsM: the per-query table lives in global memory, one
  // [m][256] region per work-group, and the work-groups take the queries in turn.
  float* lut_global;  // [gridDim.x][m][256], or null: the table is in LDS
  // Block-buffer scan whose candidate buffer would not fit LDS next to the rest: one cand_cap-key
  // region of global memory per work-group (the same bounded grid).
  uint64_t* cand_global;  // [gridDim.x][cand_cap], or null: the buffer is in LDS
};

/// Certificate of an approximate selection (mode pre). The scan kept the keep_sel best candidates by
/// approximate score, the last at a_last, so every other admitted code scores at least a_last, and
/// its exact sum at least a_last - delta. When the keep-th smallest exact sum of the selection lies
/// strictly below that, no unselected code can enter the best keep. A complete selection (no queue
/// cut or compaction ever dropped a candidate, and the selection holds all that were kept) holds
/// every admitted code and needs no check.
__device__ __forceinline__ bool adc_selection_certified(bool complete, float a_last, float r_keep, float delta) {
  if (complete) return true;
  return static_cast<double>(r_keep) < static_cast<double>(a_last) - static_cast<double>(delta);
}

/// Ascending bitonic sort of s[0, n) (n a power of two) by all 256 threads.
__device__ void block_sort_u64(uint64_t* s, uint32_t n) {
  for (uint32_t size = 2; size <= n; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (uint32_t i = threadIdx.x; i < n / 2; i += blockDim.x) {
        const uint32_t lo = 2 * i - (i & (stride - 1));
        const uint32_t hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t a = s[lo], b = s[hi];
        if ((a > b) == up) {
          s[lo] = b;
          s[hi] = a;
        }
      }
    }
  }
  __syncthreads();
}

__device__ __forceinline__ uint32_t pow2_at_least(uint32_t v) {
  uint32_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

/// Loads the mp code bytes of position pos as dwords.
template <int MPW>
__device__ __forceinline__ void load_code(const uint8_t* codes, uint64_t pos, uint32_t mp, uint32_t (&w)[MPW]) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(codes + pos * mp);
  if (mp % 16 == 0) {
#pragma unroll
    for (int i = 0; i < MPW; i += 4) {
      if (4 * i < static_cast<int>(mp)) {
        const uint4 v = *reinterpret_cast<const uint4*>(p + i);
        w[i] = v.x;
        if (i + 1 < MPW) w[i + 1] = v.y;
        if (i + 2 < MPW) w[i + 2] = v.z;
        if (i + 3 < MPW) w[i + 3] = v.w;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < MPW; ++i) {
      if (4 * i < static_cast<int>(mp)) w[i] = p[i];
    }
  }
}

/// sum_j table[j*256 + code_j] in order of j (ProductQuantizer::adc, src/product_quantizer.cc:188-192).
template <int MPW>
__device__ __forceinline__ float adc_sum(const float* lut, const uint32_t (&w)[MPW], uint32_t m) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4 * MPW; ++j) {
    if (j < static_cast<int>(m)) {
      const uint32_t c = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      s = s + lut[j * 256 + c];
    }
  }
  return s;
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

/// The code bytes [j0, j0 + 4 * MPW) of position pos as MPW dwords (zeros past the code's mp bytes).
template <int MPW>
__device__ __forceinline__ void load_code_chunk(const uint8_t* codes, uint64_t pos, uint32_t mp, uint32_t j0,
                                                uint32_t (&w)[MPW]) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(codes + pos * mp + j0);
  const int left = static_cast<int>(mp - j0);
  if (mp % 16 == 0) {
#pragma unroll
    for (int i = 0; i < MPW; i += 4) {
      if (4 * i < left) {
        const uint4 v = *reinterpret_cast<const uint4*>(p + i);
        w[i] = v.x;
        if (i + 1 < MPW) w[i + 1] = v.y;
        if (i + 2 < MPW) w[i + 2] = v.z;
        if (i + 3 < MPW) w[i + 3] = v.w;
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (i + u < MPW) w[i + u] = 0u;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < MPW; ++i) w[i] = 4 * i < left ? p[i] : 0u;
  }
}

/// Code bytes of position pos as MPW dwords. FULL (mp == 4 * MPW): the code in 16-byte pieces and
/// one 4-, 8- or 12-byte tail, each a single load (rows are only 4-byte aligned when mp is not a
/// multiple of 16, and gfx950's global loads take any width at 4-byte alignment: a 28-byte code is
/// two loads rather than seven). Otherwise dword loads of the mp bytes and zeros after them.
template <int MPW, bool FULL>
__device__ __forceinline__ void load_code_padded(const uint8_t* codes, uint64_t pos, uint32_t mp, uint32_t (&w)[MPW]) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(codes + pos * mp);
  if constexpr (FULL) {
    constexpr int kTail = MPW % 4, kHead = MPW - kTail;
#pragma unroll
    for (int i = 0; i < kHead; i += 4) {
      u32x4 v;
      __builtin_memcpy(&v, p + i, sizeof(v));
      w[i] = v.x;
      w[i + 1] = v.y;
      w[i + 2] = v.z;
      w[i + 3] = v.w;
    }
    if constexpr (kTail == 3) {
      u32x3 v;
      __builtin_memcpy(&v, p + kHead, sizeof(v));
      w[kHead] = v.x;
      w[kHead + 1] = v.y;
      w[kHead + 2] = v.z;
    } else if constexpr (kTail == 2) {
      u32x2 v;
      __builtin_memcpy(&v, p + kHead, sizeof(v));
      w[kHead] = v.x;
      w[kHead + 1] = v.y;
    } else if constexpr (kTail == 1) {
      w[kHead] = p[kHead];
    }
  } else {
#pragma unroll
    for (int i = 0; i < MPW; ++i) w[i] = 4 * i < static_cast<int>(mp) ? p[i] : 0u;
  }
}

/// sum_j table[j*256 + code_j] over all 4 * MPW table rows in order of j; rows past m hold zeros
/// (and so do the code bytes past m), and adding +0.0 leaves the reference's sum unchanged.
template <int MPW>
__device__ __forceinline__ float adc_sum_rows(const float* lut, const uint32_t (&w)[MPW]) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4 * MPW; ++j) {
    const uint32_t c = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
    s = s + lut[j * 256 + c];
  }
  return s;
}

/// The block-buffer scan of query q by one block of kScanThreads threads.
template <int MPW>
__device__ void ivf_scan_query(const ScanArgs& a, const uint32_t q) {
  extern __shared__ __attribute__((aligned(16))) unsigned char s_raw[];
  // [cand_cap]: in LDS, or in this work-group's region of global memory for large selections
  uint64_t* s_cand = a.cand_global ? a.cand_global + static_cast<uint64_t>(blockIdx.x) * a.cand_cap
                                   : reinterpret_cast<uint64_t*>(s_raw);
  uint64_t* s_pstart = reinterpret_cast<uint64_t*>(s_raw) + (a.cand_global ? 0u : a.cand_cap);  // [nprobe + 1]
  uint32_t* s_plist = reinterpret_cast<uint32_t*>(s_pstart + a.nprobe + 1);    // [nprobe]
  // [m][256]: in LDS, or in this work-group's region of global memory for m above kScanMaxLdsM
  float* s_lut = a.lut_global ? a.lut_global + static_cast<uint64_t>(blockIdx.x) * a.m * 256
                              : reinterpret_cast<float*>(s_plist + ((a.nprobe + 1) & ~1u));
  __shared__ uint32_t s_count;
  __shared__ uint64_t s_thr;
  __shared__ uint32_t s_dropped;  // a compaction dropped candidates

  const int tid = threadIdx.x;
  const float* qv = a.Q + static_cast<uint64_t>(q) * a.dim;
  const float* qscore = a.scores + static_cast<uint64_t>(q) * a.nlist;
  const uint32_t table = a.m * 256;
  constexpr uint32_t kChunk = 4 * MPW;  // sub-spaces per pass over a code
  // sum_j table[j][c_j] of position pos in order of j (ProductQuantizer::adc), kChunk at a time.
  auto adc_pos = [&](uint64_t pos) -> float {
    float sum = 0.0f;
    for (uint32_t j0 = 0; j0 < a.m; j0 += kChunk) {
      uint32_t w[MPW];
      load_code_chunk<MPW>(a.codes, pos, a.mp, j0, w);
      const float* lut = s_lut + j0 * 256;
#pragma unroll
      for (int j = 0; j < static_cast<int>(kChunk); ++j) {
        if (j0 + j < a.m) {
          const uint32_t c = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
          sum = sum + lut[j * 256 + c];
        }
      }
    }
    return sum;
  };
  // sum_j (pre[l][j][c_j] + table[j][c_j]) in order of j (src/ivfpq_index.cc:334-346).
  auto pre_pos = [&](uint64_t pos, const float* pre) -> float {
    float sum = 0.0f;
    for (uint32_t j0 = 0; j0 < a.m; j0 += kChunk) {
      uint32_t w[MPW];
      load_code_chunk<MPW>(a.codes, pos, a.mp, j0, w);
      const float* lut = s_lut + j0 * 256;
      const float* pr = pre + j0 * 256;
#pragma unroll
      for (int j = 0; j < static_cast<int>(kChunk); ++j) {
        if (j0 + j < a.m) {
          const uint32_t c = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
          sum = sum + (pr[j * 256 + c] + lut[j * 256 + c]);
        }
      }
    }
    return sum;
  };

  // Per-query table (src/ivfpq_index.cc:309-318): <q_j, C_{j,c}> in order of t, times -2 for L2.
  if (a.mode != kModeResidual && !a.exact_all) {
    for (uint32_t e = tid; e < table; e += kScanThreads) {
      const uint32_t j = e / 256, c = e % 256;
      const float* cb = a.cbt + static_cast<uint64_t>(j) * a.dsub * 256 + c;
      const float* qj = qv + static_cast<uint64_t>(j) * a.dsub;
      float v = 0.0f;
      for (uint32_t t = 0; t < a.dsub; ++t) v = v + qj[t] * cb[t * 256];
      s_lut[e] = a.mode == kModePre ? v * -2.0f : v;
    }
  }
  // Probed lists and their flattened start offsets.
  if (tid == 0) {
    uint64_t acc = 0;
    for (uint32_t p = 0; p < a.nprobe; ++p) {
      const uint32_t l = a.probes[static_cast<uint64_t>(q) * a.nprobe + p];
      s_plist[p] = l;
      s_pstart[p] = acc;
      acc += a.off[l + 1] - a.off[l];
    }
    s_pstart[a.nprobe] = acc;
    s_count = 0;
    s_thr = ~0ull;
    s_dropped = 0;
  }
  __syncthreads();

  const uint32_t keep_sel = a.keep_sel;
  // Keeps the keep_sel smallest keys of the buffer and tightens the append threshold.
  auto compact = [&]() {
    __syncthreads();
    const uint32_t cnt = min(s_count, a.cand_cap);
    const uint32_t n2 = pow2_at_least(max(cnt, 2u));
    for (uint32_t i = cnt + tid; i < n2; i += kScanThreads) s_cand[i] = ~0ull;
    block_sort_u64(s_cand, n2);
    if (tid == 0) {
      const uint32_t kept = min(cnt, keep_sel);
      if (cnt > keep_sel) s_dropped = 1;
      s_count = kept;
      if (kept == keep_sel && kept > 0) s_thr = min(s_thr, s_cand[kept - 1]);
    }
    __syncthreads();
  };
  auto offer = [&](float dist, uint64_t pos) {
    dist = dist == dist ? dist : __builtin_huge_valf();
    const uint64_t key = make_key(dist, static_cast<uint32_t>(pos));
    if (key < s_thr) {
      const uint32_t slot = atomicAdd(&s_count, 1u);
      if (slot < a.cand_cap) s_cand[slot] = key;
    }
  };

  if (a.mode != kModeResidual || a.exact_all) {
    // All probed lists as one sequence, dealt round-robin to the threads.
    const uint64_t total = s_pstart[a.nprobe];
    uint32_t p = 0;
    for (uint64_t base_v = 0; base_v < total; base_v += static_cast<uint64_t>(kScanThreads) * kScanRound) {
#pragma unroll
      for (int r = 0; r < kScanRound; ++r) {
        const uint64_t v = base_v + static_cast<uint64_t>(r) * kScanThreads + tid;
        if (v < total) {
          while (s_pstart[p + 1] <= v) ++p;
          const uint32_t l = s_plist[p];
          const uint64_t pos = a.off[l] + (v - s_pstart[p]);
          if (!a.bitmap || ((a.bitmap[pos >> 6] >> (pos & 63)) & 1ull)) {
            if (a.exact_all) {
              // Refine over every stored vector: the re-ranking distance of the refine step.
              const float* x = a.vec + pos * a.dim;
              offer(a.mode == kModeIp ? 1.0f - exact_dot(qv, x, a.dim) : exact_l2sqr(qv, x, a.dim), pos);
              continue;
            }
            const float score = qscore[l];
            float dist;
            if (a.mode == kModeIp) {
              dist = 1.0f - (-score + adc_pos(pos));  // base = <q, c> (src/ivfpq_index.cc:333,346)
            } else if (a.exact_pre) {
              // The reference's sum: table entry pre + qtab in order of j, plus ||q - c||^2.
              dist = score + pre_pos(pos, a.pre + static_cast<uint64_t>(l) * table);
            } else {
              dist = score + (a.t1[pos] + adc_pos(pos));
            }
            offer(dist, pos);
          }
        }
      }
      __syncthreads();
      if (s_count + kScanThreads * kScanRound > a.cand_cap) compact();
    }
  } else {
    // L2 without the precomputed table: a residual table per list (src/ivfpq_index.cc:338-342).
    for (uint32_t p = 0; p < a.nprobe; ++p) {
      const uint32_t l = s_plist[p];
      const uint64_t b = a.off[l], len = a.off[l + 1] - b;
      if (len == 0) continue;
      __syncthreads();
      const float* cl = a.cent + static_cast<uint64_t>(l) * a.dim;
      for (uint32_t e = tid; e < table; e += kScanThreads) {
        const uint32_t j = e / 256, c = e % 256;
        const float* cb = a.cbt + static_cast<uint64_t>(j) * a.dsub * 256 + c;
        float v = 0.0f;
        for (uint32_t t = 0; t < a.dsub; ++t) {
          const uint32_t dj = j * a.dsub + t;
          const float r = qv[dj] - cl[dj];
          const float d = r - cb[t * 256];
          v = v + d * d;
        }
        s_lut[e] = v;
      }
      __syncthreads();
      for (uint64_t i0 = 0; i0 < len; i0 += static_cast<uint64_t>(kScanThreads) * kScanRound) {
#pragma unroll
        for (int r = 0; r < kScanRound; ++r) {
          const uint64_t i = i0 + static_cast<uint64_t>(r) * kScanThreads + tid;
          if (i < len) {
            const uint64_t pos = b + i;
            if (!a.bitmap || ((a.bitmap[pos >> 6] >> (pos & 63)) & 1ull)) {
              offer(0.0f + adc_pos(pos), pos);
            }
          }
        }
        __syncthreads();
        if (s_count + kScanThreads * kScanRound > a.cand_cap) compact();
      }
    }
  }
  compact();
  uint32_t cnt = s_count;  // sorted ascending, <= keep_sel

  auto list_pos = [&](uint64_t pos) {
    uint32_t p = 0;
    while (p + 1 < a.nprobe && !(a.off[s_plist[p]] <= pos && pos < a.off[s_plist[p] + 1])) ++p;
    return s_plist[p];
  };

  // Exact re-score of the approximate ranking (L2 with the precomputed table): the reference's
  // table entry pre + qtab, summed in order of j, plus ||q - c||^2 (src/ivfpq_index.cc:334-346).
  if (a.mode == kModePre && !a.exact_all && !a.exact_pre) {
    const uint32_t selected = cnt;
    const uint64_t last = s_cand[cnt > 0 ? cnt - 1 : 0];
    __syncthreads();
    for (uint32_t i = tid; i < cnt; i += kScanThreads) {
      const uint32_t pos = static_cast<uint32_t>(s_cand[i]);
      const uint32_t l = list_pos(pos);
      float dist = qscore[l] + pre_pos(pos, a.pre + static_cast<uint64_t>(l) * table);
      dist = dist == dist ? dist : __builtin_huge_valf();
      s_cand[i] = make_key(dist, pos);
    }
    const uint32_t n2 = pow2_at_least(max(cnt, 2u));
    __syncthreads();
    for (uint32_t i = cnt + tid; i < n2; i += kScanThreads) s_cand[i] = ~0ull;
    block_sort_u64(s_cand, n2);
    cnt = min(cnt, a.keep);
    const uint64_t kth = s_cand[cnt > 0 ? cnt - 1 : 0];
    const bool certified =
        adc_selection_certified(s_dropped == 0 && selected <= keep_sel, ordered_to_float(static_cast<uint32_t>(last >> 32)),
                                ordered_to_float(static_cast<uint32_t>(kth >> 32)), a.delta[q]);
    // An uncertified query is recomputed afterwards by this kernel with exact sums (exact_pre).
    if (!certified && tid == 0) a.fallback[atomicAdd(a.nfallback, 1u)] = q;
  }

  // Exact re-ranking with the stored vectors (src/ivfpq_index.cc:139-142,363-373).
  if (a.refine) {
    for (uint32_t i = tid; i < cnt; i += kScanThreads) {
      const uint32_t pos = static_cast<uint32_t>(s_cand[i]);
      const float* x = a.vec + static_cast<uint64_t>(pos) * a.dim;
      const float e = a.mode == kModeIp ? 1.0f - exact_dot(qv, x, a.dim) : exact_l2sqr(qv, x, a.dim);
      s_cand[i] = make_key(e, pos);
    }
    const uint32_t n2 = pow2_at_least(max(cnt, 2u));
    __syncthreads();
    for (uint32_t i = cnt + tid; i < n2; i += kScanThreads) s_cand[i] = ~0ull;
    block_sort_u64(s_cand, n2);
  }

  const uint32_t nout = min(cnt, a.k);
  for (uint32_t j = tid; j < a.k; j += kScanThreads) {
    uint64_t ref = QVH_EMPTY_REF;
    float dist = __builtin_huge_valf();
    if (j < nout) {
      const uint64_t key = s_cand[j];
      const uint32_t pos = static_cast<uint32_t>(key);
      const uint32_t l = list_pos(pos);
      ref = (static_cast<uint64_t>(l) << 32) | (pos - a.off[l]);
      dist = ordered_to_float(static_cast<uint32_t>(key >> 32));
    }
    a.out_refs[static_cast<uint64_t>(q) * a.k + j] = ref;
    a.out_dist[static_cast<uint64_t>(q) * a.k + j] = dist;
  }
}

/// Block b scans query b; with a query list, the blocks take the listed queries in turn.
template <int MPW>
__global__ void __launch_bounds__(kScanThreads) ivf_scan_kernel(ScanArgs a) {
  if (!a.qlist && (a.lut_global || a.cand_global)) {
    // Tables or candidate buffers in global memory: a bounded grid, the work-groups taking the
    // queries in turn.
    for (uint32_t q = blockIdx.x; q < a.nq; q += gridDim.x) {
      ivf_scan_query<MPW>(a, q);
      __syncthreads();  // the next query reuses the block's LDS and table region
    }
    return;
  }
  if (!a.qlist) {
    ivf_scan_query<MPW>(a, blockIdx.x);
    return;
  }
  const uint32_t n = *a.qcount;
  for (uint32_t b = blockIdx.x; b < n; b += gridDim.x) {
    ivf_scan_query<MPW>(a, a.qlist[b]);
    __syncthreads();  // the next query reuses the block's LDS
  }
}

// ---- search: the streaming scan (approximate ADC in LDS, wave-private candidate queues) ----------
//
// One work-group of eight waves per query. The m x 256 table sits in LDS; the probed lists are
// walked as one flattened sequence dealt round-robin to the 512 lanes, kStreamCodes codes per lane
// in flight. Per-probe data (list start, probe key) lives in LDS and, while a lane stays in one
// list, in registers, so a code costs two 16-byte loads, one 4-byte term load and m LDS lookups.
// Candidates below the query's running threshold go to a queue private to their wave (no block
// barrier and no atomics on the append path); a full queue is sorted inside the wave and cut to
// keep_sel, and its keep_sel-th key tightens the threshold shared by the eight waves (each such key
// bounds the query's final keep_sel-th key from above). At the end the wave lists are merged and
// the keep_sel best re-scored exactly (L2 with the precomputed table) and re-ranked against the
// stored vectors (refine) before the block writes the query's results.

#ifndef QVH_STREAM_ROT
#define QVH_STREAM_ROT 0
#endif
// Default waves per streaming block: 4 with 128- or 192-entry wave queues (four blocks of ~37 KB
// LDS per CU, 128 registers per lane), 8 with 256-entry queues (three blocks of ~49 KB per CU, 80
// registers), with 512-entry queues for candidate sets of 129..256 (two blocks of ~66 KB per CU)
// or with 1024-entry queues for 257..512 (one block of ~98 KB per CU, codes of up to 32 bytes).
// The host also runs 256-entry queues on 4 waves (inner product and cosine).
template <int CAP>
constexpr int stream_waves() { return CAP <= 192 ? 4 : 8; }
constexpr uint32_t kStreamMaxProbes = 256;
constexpr uint32_t kStreamMaxSel = 512;
constexpr uint32_t kStreamMaxM = 64;  // code bytes of the widest streaming kernel
// Slices per query of a batch smaller than one resident generation of blocks.
constexpr uint64_t kMaxSlices = 16;

/// Table entry (j, c) of the per-query table, in the reference's order (sum over t, then the
/// factor -2 for L2, src/ivfpq_index.cc:315-317 and src/product_quantizer.cc:180-186).
__device__ __forceinline__ float table_entry(const float* qv, const float* cbt, uint32_t dsub, uint32_t j,
                                             uint32_t c, bool l2) {
  const float* cb = cbt + static_cast<uint64_t>(j) * dsub * 256 + c;
  const float* qj = qv + static_cast<uint64_t>(j) * dsub;
  float v = 0.0f;
  for (uint32_t t = 0; t < dsub; ++t) v = v + qj[t] * cb[t * 256];
  return l2 ? v * -2.0f : v;
}

/// delta[q] bounds |approximate - exact| for every code the query's L2 scan with the precomputed
/// table can meet. The scan sums a = score + (t1 + sum_j qtab[j][c_j]) (t1 = sum_j pre[l][j][c_j]
/// in double, rounded once), the reference r = score + sum_j (pre[l][j][c_j] + qtab[j][c_j]), both
/// in order of j. With B = |score_l|, P = sum_j |pre|, T = sum_j |qtab| over the code's terms, the
/// standard bound gamma_m on a sum of m rounded terms gives |a - V| <= (m + 2) u T + 3 u P + u B and
/// |r - V| <= (m + 2) u (P + T) + u B for the exact value V, so |a - r| <= (2m + 5) u (B + P + T)
/// up to O(u^2). delta takes (2m + 16) u (max over probed lists of |score_l| + pmax[l], plus
/// T_q), u = 2^-24, where T_q = 2 (1 + 2^-20) sum_j ||q_j|| cmax[j] bounds sum_j |qtab[j][c_j]|
/// for every code: qtab[j][c] = -2 <q_j, C_jc> is a sum of dsub rounded products, so by
/// Cauchy-Schwarz its magnitude is at most 2 (1 + dsub u) ||q_j|| ||C_jc||, and cmax[j] is the
/// largest ||C_jc||. One wave per query.
__global__ void __launch_bounds__(256) adc_bound_kernel(const float* __restrict__ Q, uint32_t nq, uint32_t dim,
                                                        uint32_t m, uint32_t dsub, const float* __restrict__ cmax,
                                                        const float* __restrict__ scores, uint32_t nlist,
                                                        const uint32_t* __restrict__ probes, uint32_t nprobe,
                                                        const float* __restrict__ pmax, float* __restrict__ delta,
                                                        uint32_t* __restrict__ fallback_count) {
  const int lane = threadIdx.x & 63;
  const uint32_t q = blockIdx.x * 4 + (threadIdx.x >> 6);
  // The scan's count of uncertified queries starts at zero (the previous search's kernels, on the
  // same stream, are done with it).
  if (blockIdx.x == 0 && threadIdx.x == 0) *fallback_count = 0u;
  if (q >= nq) return;  // whole wave
  float bp = 0.0f;
  for (uint32_t p = lane; p < nprobe; p += 64) {
    const uint32_t l = probes[static_cast<uint64_t>(q) * nprobe + p];
    bp = fmaxf(bp, fabsf(scores[static_cast<uint64_t>(q) * nlist + l]) + pmax[l]);
  }
  const float d = adc_delta(Q + static_cast<uint64_t>(q) * dim, m, dsub, cmax, bp);
  if (lane == 0) delta[q] = d;
}

/// cmax[j] = max_c ||codebook[j][c]||, computed in double and rounded up. One thread per sub-space.
__global__ void codeword_norm_kernel(const float* __restrict__ cb, uint32_t m, uint32_t dsub,
                                     float* __restrict__ cmax) {
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= m) return;
  double best = 0.0;
  for (uint32_t c = 0; c < 256; ++c) {
    const float* w = cb + (static_cast<uint64_t>(j) * 256 + c) * dsub;
    double s = 0.0;
    for (uint32_t t = 0; t < dsub; ++t) s += static_cast<double>(w[t]) * static_cast<double>(w[t]);
    best = fmax(best, sqrt(s));
  }
  const double v = best * (1.0 + 1e-12);
  const float f = static_cast<float>(v);
  cmax[j] = static_cast<double>(f) < v ? __uint_as_float(__float_as_uint(f) + 1u) : f;
}

// Bank-rotated table lookups (the L2 scan with the precomputed table). The table is laid out
// [c][R] (R = 4 * MPW rows, R <= 32), so entry (j, c) sits in bank j (mod the 64 LDS banks), and
// lane l visits the sub-spaces of its code in the order j = (l + s) mod R, s = 0..R-1: in every
// step the lanes of a half-wave read R distinct banks whatever their codes. Plain [j][256] lookups
// hit random banks, and their conflicts bound the scan; rotated ones run about 1.5x as many
// lookups per clock. The sum runs in a lane-dependent order, so it is an approximation of the
// reference's in-order sum (the scan's candidates are re-scored exactly afterwards).

/// v_cndmask_b32 with a lane mask in SGPRs: mask bit set -> b, else a. An opaque instruction, so
/// the three-stage rotation below stays three stages of selects.
__device__ __forceinline__ uint32_t select_lanes(uint32_t a, uint32_t b, uint64_t mask) {
  uint32_t r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(mask));
  return r;
}

/// Rotates this lane's code (MPW dwords) left by rot = 4 * D + b bytes: byte s of the result is
/// byte (s + rot) mod 4*MPW. D's bits arrive as lane masks (stage k moves by k dwords), b as a
/// register.
template <int MPW>
__device__ __forceinline__ void rotate_code(uint32_t (&w)[MPW], const uint64_t (&stage)[3], uint32_t b) {
#pragma unroll
  for (int st = 0; st < 3; ++st) {
    constexpr int kStages = MPW >= 8 ? 3 : MPW >= 4 ? 2 : 1;
    if (st < kStages) {
      const int k = 1 << st;
      uint32_t t[MPW];
#pragma unroll
      for (int i = 0; i < MPW; ++i) t[i] = select_lanes(w[i], w[(i + k) % MPW], stage[st]);
#pragma unroll
      for (int i = 0; i < MPW; ++i) w[i] = t[i];
    }
  }
  uint32_t t[MPW];
#pragma unroll
  for (int i = 0; i < MPW; ++i) t[i] = __builtin_amdgcn_alignbyte(w[(i + 1) % MPW], w[i], b);
#pragma unroll
  for (int i = 0; i < MPW; ++i) w[i] = t[i];
}

/// sum_s table[c_s][(rot + s) mod R] over the rotated code (byte s = c_s), in order of s.
template <int MPW>
__device__ __forceinline__ float adc_sum_rotated(const float* lut, const uint32_t (&w)[MPW], uint32_t rot) {
  constexpr int R = 4 * MPW;
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const uint32_t c = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
    s = s + lut[c * R + ((rot + j) & (R - 1))];
  }
  return s;
}

template <int MPW, bool FULL, int CAP, bool ROT, int W>
__device__ __forceinline__ void stream_scan(const ScanArgs& a) {
  constexpr int kStreamWaves = W;
  constexpr int kStreamThreads = kStreamWaves * 64;
  constexpr int QN = CAP / 64;     // queue keys per lane
  constexpr int kRows = 4 * MPW;   // table rows: the m sub-spaces, then zero rows
#ifndef QVH_STREAM_CODES
#define QVH_STREAM_CODES 2
#endif
  constexpr int kStreamCodes = QVH_STREAM_CODES;  // codes per lane per round
  extern __shared__ __attribute__((aligned(16))) unsigned char s_raw[];
  // The per-query table [kRows][256] (or [256][kRows]) is the block's static LDS for codes of up to
  // 32 bytes: it starts at LDS address 0, so each lookup's address is the code byte times 4 (one
  // SDWA shift) with the row offset in the instruction. Wider codes keep it in the dynamic segment.
  float* s_lut;
  unsigned char* s_dyn;
  if constexpr (MPW <= 8) {
    __shared__ __attribute__((aligned(16))) float s_lut_static[kRows * 256];
    s_lut = s_lut_static;
    s_dyn = s_raw;
  } else {
    s_lut = reinterpret_cast<float*>(s_raw);
    s_dyn = s_raw + kRows * 256 * sizeof(float);
  }
  uint64_t* s_queue = reinterpret_cast<uint64_t*>(s_dyn);                          // [waves][CAP]
  uint32_t* s_vstart = reinterpret_cast<uint32_t*>(s_queue + kStreamWaves * CAP);  // [nprobe + 1]
  uint32_t* s_base = s_vstart + a.nprobe + 1;  // [nprobe] list start - flattened start (mod 2^32)
  uint32_t* s_list = s_base + a.nprobe;        // [nprobe]
  float* s_score = reinterpret_cast<float*>(s_list + a.nprobe);  // [nprobe] probe keys
  // Ordered distance bits: an upper bound of the keep_sel-th distance.
  uint32_t& s_thr = *reinterpret_cast<uint32_t*>(s_score + a.nprobe);
  uint32_t* s_wcount = reinterpret_cast<uint32_t*>(s_score + a.nprobe) + 1;  // [waves]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Block -> (query slot, slice): whole queries first, then `parts` blocks per sliced query.
  uint32_t slot = blockIdx.x, part = 0;
  const bool split = blockIdx.x >= a.nwhole;
  if (split) {
    const uint32_t u = blockIdx.x - a.nwhole;
    slot = a.nwhole + u / a.parts;
    part = u % a.parts;
  }
  const uint32_t q = a.order ? a.order[slot] : slot;
  const float* qv = a.Q + static_cast<uint64_t>(q) * a.dim;
  const uint32_t m = a.m;
  const bool l2 = a.mode == kModePre;

  // Wave 0 requests the probed lists' ids, bounds and scores first: their two dependent round
  // trips then overlap the table build.
  uint32_t pf_list[4], pf_lo[4], pf_len[4];
  float pf_score[4];
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t p = lane * 4 + i;
      pf_list[i] = p < a.nprobe ? a.probes[static_cast<uint64_t>(q) * a.nprobe + p] : 0u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t p = lane * 4 + i;
      pf_lo[i] = 0;
      pf_len[i] = 0;
      pf_score[i] = 0.0f;
      if (p < a.nprobe) {
        const uint32_t l = pf_list[i];
        pf_lo[i] = static_cast<uint32_t>(a.off[l]);
        pf_len[i] = static_cast<uint32_t>(a.off[l + 1]) - pf_lo[i];
        pf_score[i] = a.scores[static_cast<uint64_t>(q) * a.nlist + l];
      }
    }
  }

  // Per-query table (src/ivfpq_index.cc:309-318).
  if (ROT) {
    // [c][kRows] layout from the c-major codebook: consecutive threads write consecutive entries
    // and read consecutive codebook rows. Rows past m are zero.
    for (uint32_t e = tid; e < 256 * kRows; e += kStreamThreads) {
      const uint32_t c = e / kRows, j = e % kRows;
      float v = 0.0f;
      if (j < m) {
        const float4 cb = *reinterpret_cast<const float4*>(a.cbc + (static_cast<uint64_t>(c) * m + j) * 4);
        const float4 qj = *reinterpret_cast<const float4*>(qv + j * 4);
        v = v + qj.x * cb.x;
        v = v + qj.y * cb.y;
        v = v + qj.z * cb.z;
        v = v + qj.w * cb.w;
        v = v * -2.0f;
      }
      s_lut[e] = v;
    }
  } else if (a.dsub == 4) {
    // Four adjacent columns c4..c4+3 of row j per lane and step: 16-byte codebook loads (a wave
    // reads 1 KB of one row contiguously) and one 16-byte LDS store per four entries; each entry is
    // summed over t in order, as before. Unrolled by 8 (all of a 32 x 256 table on 256 threads),
    // so the codebook loads go out together (unroll 2: 1.7% slower scan at nprobe 32).
#pragma unroll 8
    for (uint32_t g = tid; g < m * 64; g += kStreamThreads) {
      const uint32_t j = g >> 6, c4 = (g & 63u) * 4;
      const float* cb = a.cbt + static_cast<uint64_t>(j) * 1024 + c4;
      const float4 q4 = *reinterpret_cast<const float4*>(qv + j * 4);
      const float4 b0 = *reinterpret_cast<const float4*>(cb);
      const float4 b1 = *reinterpret_cast<const float4*>(cb + 256);
      const float4 b2 = *reinterpret_cast<const float4*>(cb + 512);
      const float4 b3 = *reinterpret_cast<const float4*>(cb + 768);
      float4 v;
      v.x = (((0.0f + q4.x * b0.x) + q4.y * b1.x) + q4.z * b2.x) + q4.w * b3.x;
      v.y = (((0.0f + q4.x * b0.y) + q4.y * b1.y) + q4.z * b2.y) + q4.w * b3.y;
      v.z = (((0.0f + q4.x * b0.z) + q4.y * b1.z) + q4.z * b2.z) + q4.w * b3.z;
      v.w = (((0.0f + q4.x * b0.w) + q4.y * b1.w) + q4.z * b2.w) + q4.w * b3.w;
      if (l2) {
        v.x = v.x * -2.0f;
        v.y = v.y * -2.0f;
        v.z = v.z * -2.0f;
        v.w = v.w * -2.0f;
      }
      *reinterpret_cast<float4*>(s_lut + j * 256 + c4) = v;
    }
  } else {
    for (uint32_t e = tid; e < m * 256; e += kStreamThreads) s_lut[e] = table_entry(qv, a.cbt, a.dsub, e >> 8, e & 255u, l2);
  }
  if (!ROT) {
    for (uint32_t e = m * 256 + tid; e < kRows * 256; e += kStreamThreads) s_lut[e] = 0.0f;
  }
  // Probed lists: lengths, then flattened starts by a wave-wide scan (nprobe <= 256).
  if (wave == 0) {
    const uint32_t(&len)[4] = pf_len;
    const uint32_t(&lo)[4] = pf_lo;
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t p = lane * 4 + i;
      if (p < a.nprobe) {
        s_list[p] = pf_list[i];
        s_score[p] = pf_score[i];
      }
      mine += len[i];
    }
    uint32_t incl = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    uint32_t start = incl - mine;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t p = lane * 4 + i;
      if (p < a.nprobe) {
        s_vstart[p] = start;
        s_base[p] = lo[i] - start;
      }
      start += len[i];
    }
    if (lane == 63) s_vstart[a.nprobe] = incl;
    if (lane == 0) s_thr = 0xFFFFFFFFu;
  }
  __syncthreads();
  const uint32_t keep_sel = a.keep_sel;
  uint64_t* queue = s_queue + wave * CAP;
  uint32_t cnt = 0;                   // wave-uniform queue fill
  float thr = __builtin_huge_valf();  // candidates need dist <= thr
  uint32_t thr_bits = 0xFFFFFFFFu;    // the same bound as ordered bits

  // Cuts the wave's queue to the entries whose distance is at most the keep_sel-th smallest one
  // (found bit by bit with wave ballots), and publishes that distance as the shared bound. Ties at
  // that distance are all kept unless that would keep more than tie_limit (>= keep_sel) entries.
  auto flush = [&](uint32_t tie_limit) {
    uint64_t k[QN];
    uint32_t d[QN];
#pragma unroll
    for (int i = 0; i < QN; ++i) {
      const uint32_t e = i * 64 + lane;
      k[i] = e < cnt ? queue[e] : ~0ull;
      d[i] = static_cast<uint32_t>(k[i] >> 32);
    }
    if (cnt <= keep_sel) return;
    uint32_t t = 0;
    for (int b = 31; b >= 0; --b) {
      const uint32_t probe = t | ((1u << b) - 1u);
      uint32_t below = 0;
#pragma unroll
      for (int i = 0; i < QN; ++i) {
        if (static_cast<uint32_t>(i * 64) < cnt) below += static_cast<uint32_t>(__popcll(__ballot(d[i] <= probe)));
      }
      if (below < keep_sel) t |= 1u << b;
    }
    // t is the keep_sel-th smallest distance (as ordered bits); keep every entry at or below it,
    // unless ties at t would keep more than tie_limit: then also find the position u such that the
    // entries below t plus the ties at t with position <= u are exactly keep_sel.
    uint32_t kept = 0, under = 0;
#pragma unroll
    for (int i = 0; i < QN; ++i) {
      if (static_cast<uint32_t>(i * 64) < cnt) {
        kept += static_cast<uint32_t>(__popcll(__ballot(d[i] <= t)));
        under += static_cast<uint32_t>(__popcll(__ballot(d[i] < t)));
      }
    }
    uint32_t u = 0xFFFFFFFFu;
    if (kept > tie_limit) {
      const uint32_t need = keep_sel - under;
      u = 0;
      for (int b = 31; b >= 0; --b) {
        const uint32_t probe = u | ((1u << b) - 1u);
        uint32_t below = 0;
#pragma unroll
        for (int i = 0; i < QN; ++i) {
          if (static_cast<uint32_t>(i * 64) < cnt) {
            below += static_cast<uint32_t>(__popcll(__ballot(d[i] == t && static_cast<uint32_t>(k[i]) <= probe)));
          }
        }
        if (below < need) u |= 1u << b;
      }
    }
    __builtin_amdgcn_wave_barrier();
    uint32_t at = 0;
#pragma unroll
    for (int i = 0; i < QN; ++i) {
      if (static_cast<uint32_t>(i * 64) < cnt) {
        const bool keepit = k[i] != ~0ull && (d[i] < t || (d[i] == t && static_cast<uint32_t>(k[i]) <= u));
        const uint64_t mk = __ballot(keepit);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mk >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mk), 0u));
        if (keepit) queue[at + below] = k[i];
        at += static_cast<uint32_t>(__popcll(mk));
      }
    }
    __builtin_amdgcn_wave_barrier();
    cnt = at;
    // t, the keep_sel-th smallest distance among the wave's candidates, bounds the query's.
    if (lane == 0) atomicMin(&s_thr, t);
    if (t < thr_bits) {
      thr_bits = t;
      thr = ordered_to_float(t);
    }
  };
  // Appends one code's candidates (at most 64) at a time and cuts the queue once it holds more than
  // flush_at = CAP - 64; a cut leaves at most CAP / 2 (keep_sel <= CAP / 2), so the queue never
  // holds more than CAP, and at least CAP / 2 - 64 candidates arrive between two cuts.
  const uint32_t flush_at = CAP - 64;
  auto offer = [&](bool pass, float d, uint32_t pos) {
    pass = pass && d <= thr;
    const uint64_t mk = __ballot(pass);
    if (mk == 0) return;
    const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mk >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mk), 0u));
    if (pass) queue[cnt + below] = make_key(d, pos);
    cnt += static_cast<uint32_t>(__popcll(mk));
    if (cnt > flush_at) flush(CAP / 2);
  };

  // This block's slice [v_lo, v_hi) of the query's flattened probed positions.
  const uint32_t total = s_vstart[a.nprobe];
  const uint32_t v_lo = split ? static_cast<uint32_t>(static_cast<uint64_t>(total) * part / a.parts) : 0u;
  const uint32_t v_hi = split ? static_cast<uint32_t>(static_cast<uint64_t>(total) * (part + 1) / a.parts) : total;
  uint32_t p = 0;
  uint32_t vend = s_vstart[1];
  uint32_t base = s_base[0];
  float score = s_score[0];
  // Software-pipelined: the codes (and t1 terms, and filter words) of round i + 1 are requested
  // before round i's table lookups, so every wave keeps a round of loads in flight while it sums.
  uint32_t npos[kStreamCodes];
  float nsc[kStreamCodes], nt1[kStreamCodes];
  bool nok[kStreamCodes];
  uint32_t nw[kStreamCodes][MPW];
  uint64_t nbits[kStreamCodes];
  auto fetch = [&](uint32_t v0) {
#pragma unroll
    for (int r = 0; r < kStreamCodes; ++r) {
      const uint32_t v = v0 + r * kStreamThreads + tid;
      nok[r] = v < v_hi;
      if (nok[r] && v >= vend) {
        do {
          ++p;
        } while (v >= s_vstart[p + 1]);
        vend = s_vstart[p + 1];
        base = s_base[p];
        score = s_score[p];
      }
      npos[r] = v + base;
      nsc[r] = score;
      const uint32_t pr = nok[r] ? npos[r] : 0u;
      load_code_padded<MPW, FULL>(a.codes, pr, a.mp, nw[r]);
      nt1[r] = l2 ? a.t1[pr] : 0.0f;
      nbits[r] = a.bitmap ? a.bitmap[pr >> 6] : ~0ull;
    }
  };
  // Rotation of this lane's codes (bank-rotated lookups): rot = lane mod kRows.
  const uint32_t rot = static_cast<uint32_t>(lane) & (kRows - 1);
  uint64_t stage[3];
#pragma unroll
  for (int st = 0; st < 3; ++st) stage[st] = __ballot(((rot >> 2) >> st) & 1u);
  if (v_lo < v_hi) fetch(v_lo);
  for (uint32_t v0 = v_lo; v0 < v_hi; v0 += kStreamThreads * kStreamCodes) {
    uint32_t pos[kStreamCodes];
    float sc[kStreamCodes], t1v[kStreamCodes];
    bool ok[kStreamCodes];
    uint32_t w[kStreamCodes][MPW];
#pragma unroll
    for (int r = 0; r < kStreamCodes; ++r) {
      pos[r] = npos[r];
      sc[r] = nsc[r];
      t1v[r] = nt1[r];
      ok[r] = nok[r] && ((nbits[r] >> (pos[r] & 63)) & 1ull);
#pragma unroll
      for (int i = 0; i < MPW; ++i) w[r][i] = nw[r][i];
    }
    if (v0 + kStreamThreads * kStreamCodes < v_hi) fetch(v0 + kStreamThreads * kStreamCodes);
    float dist[kStreamCodes];
    bool any = false;
    // The rotation as seen by this round: its table columns are recomputed per round (and shared by
    // the round's codes) rather than held in registers across the loop.
    uint32_t rot_round = rot;
    if constexpr (ROT) asm volatile("" : "+v"(rot_round));
#pragma unroll
    for (int r = 0; r < kStreamCodes; ++r) {
      float sum;
      if constexpr (ROT) {
        rotate_code<MPW>(w[r], stage, rot & 3u);
        sum = adc_sum_rotated<MPW>(s_lut, w[r], rot_round);
      } else {
        sum = adc_sum_rows<MPW>(s_lut, w[r]);
      }
      const float d = l2 ? sc[r] + (t1v[r] + sum) : 1.0f - (-sc[r] + sum);  // src/ivfpq_index.cc:333-346
      dist[r] = d == d ? d : __builtin_huge_valf();
      any = any || (ok[r] && dist[r] <= thr);
    }
    if (__ballot(any) != 0) {
#pragma unroll
      for (int r = 0; r < kStreamCodes; ++r) offer(ok[r], dist[r], pos[r]);
    }
    if (v0 == v_lo) {
      // Every wave cuts its first candidates and the block shares the tightest bound.
      flush(CAP / 2);
      __syncthreads();
    }
    // An atomic load at workgroup scope stays an LDS read; a volatile read of this reference
    // became a flat load whose wait also drained the next step's loads.
    const uint32_t shared_thr = __hip_atomic_load(&s_thr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (shared_thr < thr_bits) {
      thr_bits = shared_thr;
      thr = ordered_to_float(shared_thr);
    }
  }
  // Probe index of a position: eight probed lists tested per step (independent LDS reads).
  auto list_of = [&](uint32_t pos) {
    for (uint32_t b = 0; b + 1 < a.nprobe; b += 8) {
      uint32_t hit = 0;
#pragma unroll
      for (uint32_t i = 0; i < 8; ++i) {
        const uint32_t pl = b + i;
        if (pl < a.nprobe && pos - (s_base[pl] + s_vstart[pl]) < s_vstart[pl + 1] - s_vstart[pl]) hit |= 1u << i;
      }
      if (hit) return b + static_cast<uint32_t>(__builtin_ctz(hit));
    }
    return a.nprobe - 1;
  };
  // Exact re-score of one approximate candidate (L2 with the precomputed table): the reference's
  // table entry pre + qtab, summed in order of j, plus ||q - c||^2 (src/ivfpq_index.cc:334-346).
  auto rescore = [&](uint64_t key) -> uint64_t {
    const uint32_t pos = static_cast<uint32_t>(key);
    uint32_t wc[MPW];
    load_code<MPW>(a.codes, pos, a.mp, wc);  // in flight during the list search
    const uint32_t pl = list_of(pos);
    const float* pre = a.pre + static_cast<uint64_t>(s_list[pl]) * m * 256;
    // All 4 * MPW table loads go out together. Rows past m (whole code dwords still carry up to three
    // pad bytes when m is not a multiple of four) re-read row m - 1 and are not added: the list's
    // table has exactly m rows, the next list's follow it.
    float pv[4 * MPW];
#pragma unroll
    for (int j = 0; j < 4 * MPW; ++j) {
      const int jr = min(j, static_cast<int>(m) - 1);
      const uint32_t c = (wc[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      pv[j] = pre[jr * 256 + c];
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 4 * MPW; ++j) {
      const uint32_t c = (wc[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      if (j < static_cast<int>(m)) sum = sum + (pv[j] + s_lut[ROT ? c * kRows + j : j * 256 + c]);
    }
    float d = s_score[pl] + sum;
    d = d == d ? d : __builtin_huge_valf();
    return make_key(d, pos);
  };
  // Re-ranking key of a candidate (refine): its exact distance to the stored vector, summed in the
  // reference's order (src/ivfpq_index.cc:139-142,363-373).
  auto refine_key = [&](uint32_t pos) -> uint64_t {
    const float* x = a.vec + static_cast<uint64_t>(pos) * a.dim;
    const float e = l2 ? exact_l2sqr(qv, x, a.dim) : 1.0f - exact_dot(qv, x, a.dim);
    return make_key(e, pos);
  };
  // Result j of the query: the list ref and distance of `key`, or an empty slot.
  auto emit = [&](uint32_t j, bool full_slot, uint64_t key) {
    uint64_t ref = QVH_EMPTY_REF;
    float d = __builtin_huge_valf();
    if (full_slot) {
      const uint32_t pos = static_cast<uint32_t>(key);
      const uint32_t pl = list_of(pos);
      ref = (static_cast<uint64_t>(s_list[pl]) << 32) | (pos - (s_base[pl] + s_vstart[pl]));
      d = ordered_to_float(static_cast<uint32_t>(key >> 32));
    }
    a.out_refs[static_cast<uint64_t>(q) * a.k + j] = ref;
    a.out_dist[static_cast<uint64_t>(q) * a.k + j] = d;
  };
  // Blocks with 256- or 512-entry queues cut only a list longer than CAP / 2 (a key a cut would
  // drop has keep_sel better ones in its own list). Four-wave blocks with smaller queues always
  // cut, which keeps wave 0's sort below at <= 4 keep_sel keys.
  if constexpr (kStreamWaves == 4 && CAP <= 192) {
    flush(64);
    // Single-wave finish (four waves, k and keep_sel <= 64): the four cut lists (<= 64 keys each)
    // are packed in LDS, then wave 0 alone sorts, re-scores and emits them in registers, with no
    // further block barrier.
    const uint64_t mine = static_cast<uint32_t>(lane) < cnt ? queue[lane] : ~0ull;
    if (lane == 0) s_wcount[wave] = cnt;
    __syncthreads();
    uint32_t before = 0, merged = 0;
#pragma unroll
    for (int w2 = 0; w2 < kStreamWaves; ++w2) {
      const uint32_t c = s_wcount[w2];
      if (w2 < wave) before += c;
      merged += c;
    }
    if (static_cast<uint32_t>(lane) < cnt) s_queue[before + lane] = mine;
    __syncthreads();
    if (wave != 0) return;
    // The `count` smallest of the `total` (<= 256) keys packed at s_queue[0, total), ascending:
    // key i sits in lane i of the result (count <= 64).
    auto wave_smallest = [&](uint32_t total, uint32_t count) -> uint64_t {
      uint64_t kk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t e = i * 64 + lane;
        kk[i] = e < total ? s_queue[e] : ~0ull;
      }
      if (total <= 64) {
        uint64_t t[1] = {kk[0]};
        wave_sort<1>(t);
        kk[0] = t[0];
      } else if (total <= 128) {
        uint64_t t[2] = {kk[0], kk[1]};
        wave_sort<2>(t);
        kk[0] = t[0];
      } else {
        wave_sort<4>(kk);
      }
      return static_cast<uint32_t>(lane) < count ? kk[0] : ~0ull;
    };
    uint32_t cnt_f = min(merged, keep_sel);
    uint64_t key = wave_smallest(merged, cnt_f);
    bool certified = true;
    if (l2) {
      const uint64_t last = __shfl(key, static_cast<int>(cnt_f > 0 ? cnt_f - 1 : 0), 64);
      if (static_cast<uint32_t>(lane) < cnt_f) key = rescore(key);
      uint64_t t[1] = {key};
      wave_sort<1>(t);
      key = t[0];
      cnt_f = min(cnt_f, a.keep);
      const uint64_t kth = __shfl(key, static_cast<int>(cnt_f > 0 ? cnt_f - 1 : 0), 64);
      // No wave ever cut its queue (s_thr untouched) and the selection took every kept key.
      const bool complete = merged <= keep_sel && s_thr == 0xFFFFFFFFu;
      certified = adc_selection_certified(complete, ordered_to_float(static_cast<uint32_t>(last >> 32)),
                                          ordered_to_float(static_cast<uint32_t>(kth >> 32)), a.delta[q]);
    }
    if (split) {
      // The slice's best keep keys and its count (bit 31: uncertified) go out as agent-scope atomic
      // stores; every lane then releases them at agent scope before lane 0 counts the slice done,
      // and the last slice of the query acquires at agent scope before it reads the lists.
      const uint32_t tq = slot - a.nwhole;
      uint64_t* lists = a.part_keys + static_cast<uint64_t>(tq) * a.parts * a.keep;
      if (static_cast<uint32_t>(lane) < cnt_f) {
        __hip_atomic_store(&lists[static_cast<uint64_t>(part) * a.keep + lane], key, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      if (lane == 0) {
        __hip_atomic_store(&a.part_cnt[tq * a.parts + part], cnt_f | (certified ? 0u : 0x80000000u), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __builtin_amdgcn_wave_barrier();
      uint32_t done = 0;
      if (lane == 0) done = __hip_atomic_fetch_add(&a.part_done[tq], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      if (__shfl(done, 0, 64) != a.parts - 1) return;
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      uint32_t all = 0;
      certified = true;
      for (uint32_t pi = 0; pi < a.parts; ++pi) {
        const uint32_t cw = __hip_atomic_load(&a.part_cnt[tq * a.parts + pi], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t c = cw & 0x7FFFFFFFu;
        certified = certified && (cw >> 31) == 0;
        for (uint32_t i = lane; i < c; i += 64) {
          s_queue[all + i] = __hip_atomic_load(&lists[static_cast<uint64_t>(pi) * a.keep + i], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
        }
        all += c;
      }
      __builtin_amdgcn_wave_barrier();
      cnt_f = min(all, a.keep);
      key = wave_smallest(all, cnt_f);
      if (lane == 0) __hip_atomic_store(&a.part_done[tq], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // An uncertified query is recomputed by the block-buffer scan with exact sums, which runs after
    // this kernel and overwrites its results.
    if (!certified && lane == 0) a.fallback[atomicAdd(a.nfallback, 1u)] = q;
    if (a.refine) {
      // One candidate per lane, then a register sort by the exact distance.
      uint64_t t[1] = {static_cast<uint32_t>(lane) < cnt_f ? refine_key(static_cast<uint32_t>(key)) : ~0ull};
      wave_sort<1>(t);
      key = t[0];
    }
    if (static_cast<uint32_t>(lane) < a.k) emit(lane, static_cast<uint32_t>(lane) < min(cnt_f, a.k), key);
    return;
  }
  // Queues of 256, 512 or 1024 entries (keep_sel <= CAP / 2): each wave sorts its list (<= CAP / 2
  // keys, NK per lane) in registers; log2(waves) rounds of pairwise merges then keep the CAP / 2
  // smallest: the elementwise minimum of one sorted list and the other reversed holds the CAP / 2
  // smallest of both as a bitonic sequence, which a register bitonic merge orders. Wave 0's region
  // ends with the block's CAP / 2 smallest, sorted. (Blocks with smaller queues returned above;
  // this is compiled for them too but never reached.)
  uint32_t merged = 0;
  if constexpr (CAP >= 256) {
  if (cnt > static_cast<uint32_t>(CAP / 2)) flush(CAP / 2);
  constexpr int NK = CAP / 128;
  constexpr int kList = CAP / 2;
  uint64_t mine[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) mine[i] = static_cast<uint32_t>(i * 64 + lane) < cnt ? queue[i * 64 + lane] : ~0ull;
  wave_sort<NK>(mine);
#pragma unroll
  for (int i = 0; i < NK; ++i) queue[i * 64 + lane] = mine[i];
  if (lane == 0) s_wcount[wave] = cnt;
  __syncthreads();
#pragma unroll
  for (int w2 = 0; w2 < kStreamWaves; ++w2) merged += s_wcount[w2];
#pragma unroll
  for (int step = 1; step < kStreamWaves; step *= 2) {
    if (wave % (2 * step) == 0) {
      const uint64_t* other = s_queue + (wave + step) * CAP;
#pragma unroll
      for (int i = 0; i < NK; ++i) {
        const uint64_t o = other[kList - 1 - (i * 64 + lane)];
        mine[i] = o < mine[i] ? o : mine[i];
      }
      wave_merge<NK>(mine);
#pragma unroll
      for (int i = 0; i < NK; ++i) queue[i * 64 + lane] = mine[i];
    }
    __syncthreads();
  }
  }
  uint32_t cnt_f = min(merged, keep_sel);
  bool certified = true;
  // Sorts s_queue[0, count) (count <= CAP / 2, at most 512) ascending in wave 0's registers (no
  // block barriers inside the sort); slots past count read as empty. The block waits before and
  // after.
  auto sort_front = [&](uint32_t count) {
    __syncthreads();
    if (wave == 0) {
      if (CAP >= 1024 && count > 256) {
        uint64_t t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = static_cast<uint32_t>(i * 64 + lane) < count ? s_queue[i * 64 + lane] : ~0ull;
        wave_sort<8>(t);
#pragma unroll
        for (int i = 0; i < 8; ++i) s_queue[i * 64 + lane] = t[i];
      } else if (count <= 128) {
        uint64_t t[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) t[i] = static_cast<uint32_t>(i * 64 + lane) < count ? s_queue[i * 64 + lane] : ~0ull;
        wave_sort<2>(t);
#pragma unroll
        for (int i = 0; i < 2; ++i) s_queue[i * 64 + lane] = t[i];
      } else {
        uint64_t t[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) t[i] = static_cast<uint32_t>(i * 64 + lane) < count ? s_queue[i * 64 + lane] : ~0ull;
        wave_sort<4>(t);
#pragma unroll
        for (int i = 0; i < 4; ++i) s_queue[i * 64 + lane] = t[i];
      }
    }
    __syncthreads();
  };

  // Exact re-score of the approximate ranking (L2 with the precomputed table): the reference's
  // table entry pre + qtab, summed in order of j, plus ||q - c||^2 (src/ivfpq_index.cc:334-346).
  if (l2) {
    const uint64_t last = s_queue[cnt_f > 0 ? cnt_f - 1 : 0];
    __syncthreads();
    if (static_cast<uint32_t>(tid) < cnt_f) s_queue[tid] = rescore(s_queue[tid]);
    sort_front(cnt_f);
    cnt_f = min(cnt_f, a.keep);
    const uint64_t kth = s_queue[cnt_f > 0 ? cnt_f - 1 : 0];
    const bool complete = merged <= keep_sel && s_thr == 0xFFFFFFFFu;
    certified = adc_selection_certified(complete, ordered_to_float(static_cast<uint32_t>(last >> 32)),
                                        ordered_to_float(static_cast<uint32_t>(kth >> 32)), a.delta[q]);
  }
  if (split) {
    // A slice leaves its (at most keep) best keys; the last slice of the query to finish merges
    // the lists (the best keep keys of the union are the best keep keys of the whole scan). The
    // lists and counts (bit 31: uncertified) go out as agent-scope atomic stores, every thread
    // releases them at agent scope before the barrier after which thread 0 counts the slice done,
    // and the merging slice acquires at agent scope before it reads them.
    const uint32_t tq = slot - a.nwhole;
    uint64_t* lists = a.part_keys + static_cast<uint64_t>(tq) * a.parts * a.keep;
    for (uint32_t i = tid; i < cnt_f; i += kStreamThreads) {
      __hip_atomic_store(&lists[static_cast<uint64_t>(part) * a.keep + i], s_queue[i], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0) {
      __hip_atomic_store(&a.part_cnt[tq * a.parts + part], cnt_f | (certified ? 0u : 0x80000000u), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
      const uint32_t before = __hip_atomic_fetch_add(&a.part_done[tq], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      s_wcount[0] = before == a.parts - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (s_wcount[0] == 0) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    uint32_t all = 0;
    certified = true;
    for (uint32_t pi = 0; pi < a.parts; ++pi) {
      const uint32_t cw = __hip_atomic_load(&a.part_cnt[tq * a.parts + pi], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t c = cw & 0x7FFFFFFFu;
      certified = certified && (cw >> 31) == 0;
      for (uint32_t i = tid; i < c; i += kStreamThreads) {
        s_queue[all + i] = __hip_atomic_load(&lists[static_cast<uint64_t>(pi) * a.keep + i], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      }
      all += c;
    }
    const uint32_t n3 = pow2_at_least(max(all, 2u));
    for (uint32_t i = all + tid; i < n3; i += kStreamThreads) s_queue[i] = ~0ull;
    for (uint32_t size = 2; size <= n3; size <<= 1) {
      for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
        __syncthreads();
        for (uint32_t i = tid; i < n3 / 2; i += kStreamThreads) {
          const uint32_t lo = 2 * i - (i & (stride - 1));
          const uint32_t hi = lo + stride;
          const bool up = (lo & size) == 0;
          const uint64_t x = s_queue[lo], y = s_queue[hi];
          if ((x > y) == up) {
            s_queue[lo] = y;
            s_queue[hi] = x;
          }
        }
      }
    }
    __syncthreads();
    cnt_f = min(all, a.keep);
    if (tid == 0) __hip_atomic_store(&a.part_done[tq], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next search
  }
  // An uncertified query is recomputed by the block-buffer scan with exact sums, which runs after
  // this kernel and overwrites its results.
  if (!certified && tid == 0) a.fallback[atomicAdd(a.nfallback, 1u)] = q;
  if (a.refine) {
    // The cnt_f best keys are s_queue[0, cnt_f) here (every thread has passed a barrier since they
    // were written). Eight lanes per candidate compute its exact distance (each lane's loads
    // coalesced with its group's), NC candidates per group at once so that every candidate's row
    // loads are in flight together (keep_sel <= CAP / 2 candidates in one pass), then a block sort
    // by the exact distance. Slots past cnt_f score the query against itself and are dropped.
    constexpr uint32_t kGroups = kStreamThreads / 8;
    constexpr int NC = static_cast<int>((CAP / 2 + kGroups - 1) / kGroups);
    for (uint32_t b = 0; b < cnt_f; b += NC * kGroups) {
      uint32_t pos[NC];
      const float* x[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint32_t i = b + c * kGroups + static_cast<uint32_t>(tid) / 8;
        pos[c] = i < cnt_f ? static_cast<uint32_t>(s_queue[i]) : 0u;
        x[c] = i < cnt_f ? a.vec + static_cast<uint64_t>(pos[c]) * a.dim : qv;
      }
      float e[NC];
      if (l2) {
        exact_group8_n<true, NC>(qv, x, a.dim, e);
      } else {
        exact_group8_n<false, NC>(qv, x, a.dim, e);
#pragma unroll
        for (int c = 0; c < NC; ++c) e[c] = 1.0f - e[c];
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint32_t i = b + c * kGroups + static_cast<uint32_t>(tid) / 8;
        if (i < cnt_f && (tid & 7) == 0) s_queue[i] = make_key(e[c], pos[c]);
      }
    }
    sort_front(cnt_f);
  }
  const uint32_t nout = min(cnt_f, a.k);
  for (uint32_t j = tid; j < a.k; j += kStreamThreads) emit(j, j < nout, s_queue[j < nout ? j : 0]);
}

// Up to 32 code bytes. W waves per block (four for queues of up to 192 entries, eight for 512,
// either for 256).
template <int MPW, bool FULL, int CAP, bool ROT = false, int W = stream_waves<CAP>()>
__global__ void __launch_bounds__(W * 64)
__attribute__((amdgpu_waves_per_eu(W == 4 || CAP == 512 ? 4 : CAP >= 1024 ? 2 : 6))) ivf_stream_kernel(ScanArgs a) {
  stream_scan<MPW, FULL, CAP, ROT, W>(a);
}

// 33 to 64 code bytes: no register cap. (ROT is not used: it keeps the template arguments after
// the code width the same as ivf_stream_kernel's, so one launch macro serves both.)
template <bool FULL, int CAP, bool ROT = false, int W = stream_waves<CAP>()>
__global__ void __launch_bounds__(W * 64) ivf_stream_wide_kernel(ScanArgs a) {
  stream_scan<16, FULL, CAP, false, W>(a);
}

void launch_nearest(bool sqdiff, const NearestArgs& a, uint32_t nsub, hipStream_t s) {
  if (a.n == 0) return;
  const dim3 grid(static_cast<unsigned>(ceil_div(a.n, kNearThreads)), nsub);
  if (sqdiff) {
    hipLaunchKernelGGL(nearest_kernel<true>, grid, dim3(kNearThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL(nearest_kernel<false>, grid, dim3(kNearThreads), 0, s, a);
  }
  QVH_HIP(hipGetLastError());
}

/// The MFMA assignment's operand for one centroid table, prepared once per table.
struct AssignTable {
  DeviceBuffer crow, aug, rmax;
  uint32_t dim = 0, dp = 0, kp = 0;
  bool ready = false;
};

/// Prepares `t` for centroids d_cent [k][dim] with in-order norms d_norms (centroid_prep_kernel).
/// Dims that are not a multiple of 4, below kAsgMinDim (PQ sub-spaces: mostly padding, and the
/// VALU kernel is fast there) or above kAsgMaxDp leave it unprepared (exact kernel only).
void prepare_assign_table(AssignTable& t, const float* d_cent, const float* d_norms, uint32_t k, uint32_t dim,
                          int max_ip, hipStream_t s) {
  t.ready = false;
  if (k == 0 || dim % 4 != 0 || dim < kAsgMinDim || dim > kAsgMaxDp) return;
  t.dim = dim;
  t.dp = (dim + 31) / 32 * 32;
  t.kp = static_cast<uint32_t>(ceil_div(k, kAsgTile) * kAsgTile);
  const uint64_t cells = static_cast<uint64_t>(t.kp) * t.dp;
  t.crow.reserve(cells * sizeof(float));
  t.aug.reserve(t.kp * sizeof(float));
  t.rmax.reserve(sizeof(float));
  hipLaunchKernelGGL(assign_rows_kernel, dim3(static_cast<unsigned>(ceil_div(cells, 256))), dim3(256), 0, s, d_cent,
                     d_norms, k, dim, t.dp, t.kp, max_ip, t.crow.as<float>(), t.aug.as<float>());
  hipLaunchKernelGGL(norm_max_kernel, dim3(1), dim3(256), 0, s, d_norms, k, t.rmax.as<float>());
  QVH_HIP(hipGetLastError());
  t.ready = true;
}

template <int DP>
void launch_assign_dp(bool l2, const AssignArgs& a, dim3 grid, hipStream_t s) {
  if (l2) {
    hipLaunchKernelGGL((assign_mfma_kernel<DP, true>), grid, dim3(kAsgThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((assign_mfma_kernel<DP, false>), grid, dim3(kAsgThreads), 0, s, a);
  }
}

/// Nearest centroids (nearest mode of `na`) of na.n points: the MFMA kernel where the table is
/// prepared and the batch is large, then the exact kernel for the points it could not certify;
/// the exact kernel for every point otherwise. `fb` is workspace (n + 1 words).
void launch_assign(const NearestArgs& na, const AssignTable& t, DeviceBuffer& fb, hipStream_t s) {
  if (na.n == 0) return;
  const bool mfma = t.ready && na.dim == t.dim && na.n >= kAsgMinPoints && na.n < 0xFFFFFFFFull &&
                    na.x_stride % 4 == 0 && reinterpret_cast<uintptr_t>(na.x) % 16 == 0;
  if (!mfma) {
    launch_nearest(false, na, 1, s);
    return;
  }
  uint32_t* list = static_cast<uint32_t*>(fb.reserve((na.n + 1) * sizeof(uint32_t)));
  hipLaunchKernelGGL(assign_reset_kernel, dim3(1), dim3(1), 0, s, list);
  AssignArgs a{};
  a.x = na.x;
  a.n = na.n;
  a.dim = na.dim;
  a.x_stride = na.x_stride;
  a.crow = t.crow.as<float>();
  a.aug = t.aug.as<float>();
  a.kp = t.kp;
  a.rmax = t.rmax.as<float>();
  a.coef = ldexpf(4.0f * static_cast<float>(t.dp + 1) + 16.0f, -24);
  a.out32 = na.out32;
  a.fb = list;
  const dim3 grid(static_cast<unsigned>(ceil_div(na.n, kAsgPoints)));
  const bool l2 = !na.max_ip;
  switch (t.dp) {
    case 32: launch_assign_dp<32>(l2, a, grid, s); break;
    case 64: launch_assign_dp<64>(l2, a, grid, s); break;
    case 96: launch_assign_dp<96>(l2, a, grid, s); break;
    default: launch_assign_dp<128>(l2, a, grid, s); break;
  }
  QVH_HIP(hipGetLastError());
  NearestArgs ex = na;
  ex.list = list;
  const uint64_t blocks = std::min<uint64_t>(na.n, 2048);
  hipLaunchKernelGGL(nearest_listed_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, ex);
  QVH_HIP(hipGetLastError());
}

}  // namespace

namespace qvh {

/// PQ codes [n][m] of n rows [n][dim] (ProductQuantizer::encode, src/product_quantizer.cc:165-171):
/// per sub-space the first nearest of the 256 codewords by the in-order sum of squared differences,
/// against the per-sub-space transposed codebook [m][dsub][256].
void launch_pq_encode(const float* d_x, uint64_t n, uint32_t dim, uint32_t m, const float* d_cbt, uint8_t* d_codes,
                      hipStream_t s) {
  NearestArgs pa{};
  pa.x = d_x;
  pa.n = n;
  pa.dim = dim / m;  // per sub-space
  pa.x_stride = dim;
  pa.x_off = 0;
  pa.ct = d_cbt;
  pa.k = 256;
  pa.out8 = d_codes;
  pa.out_stride = m;
  launch_nearest(true, pa, m, s);
}

/// Codebook [m][256][dsub] -> per sub-space transposed [m][dsub][256].
void launch_codebook_transpose(const float* d_cb, uint32_t m, uint32_t dsub, float* d_cbt, hipStream_t s) {
  hipLaunchKernelGGL(codebook_prep_kernel, dim3(static_cast<unsigned>(ceil_div(uint64_t(m) * 256 * dsub, 256))),
                     dim3(256), 0, s, d_cb, m, dsub, d_cbt);
  QVH_HIP(hipGetLastError());
}

}  // namespace qvh

/// Measurement only: bytes of PQ codes the scan must read, sum over queries and probes of
/// len(list) * m. One block; thread sums, then an LDS tree.
__global__ void __launch_bounds__(256) probed_code_bytes_kernel(const uint32_t* __restrict__ probes, uint64_t entries,
                                                                const uint64_t* __restrict__ off, uint32_t m,
                                                                uint64_t* __restrict__ out) {
  __shared__ uint64_t part[256];
  uint64_t s = 0;
  for (uint64_t i = threadIdx.x; i < entries; i += 256) {
    const uint32_t l = probes[i];
    s += off[l + 1] - off[l];
  }
  part[threadIdx.x] = s;
  __syncthreads();
  for (unsigned w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = part[0] * m;
}

// ---- handle ---------------------------------------------------------------------------------------

/// Workspace of the encode step (cells, residuals, codes of a batch being added). It has its own
/// lock and stream, apart from the search workspace: the trained state it reads never changes once
/// installed, so an add's encode runs on the device beside searches of the same handle, and only
/// the append that follows takes the handle's lock (src/ivfpq_index.cc:226-249).
struct EncodeSpace {
  std::mutex mu;
  hipStream_t stream = nullptr;
  DeviceBuffer x, assign, afb, res, codes;
};

struct qvh_ivfpq {
  uint32_t dim = 0, nlist = 0, m = 0, dsub = 0, mp = 0;
  int metric = 0;
  int store_vectors = 0;
  int device = 0;
  std::atomic<bool> trained{false};  // set once, after the trained state is on the device
  bool has_pre = false;
  uint64_t count = 0;
  std::vector<uint64_t> h_off;  // host copy of the list offsets
  DeviceBuffer cent, cent_t, cent_norm, cb, cbt, cbc, pre;
  AssignTable asg;  // the centroids as the MFMA assignment's operand
  DeviceBuffer off, codes, t1, vec;
  DeviceBuffer pmax;  // [nlist] sum_j max_c |pre[l][j][c]| (the L2 ranking's certificate)
  DeviceBuffer cmax;  // [m] largest codeword norm per sub-space (the same)
  hipStream_t stream = nullptr;
  std::mutex mu;
  EncodeSpace enc;
  DeviceBuffer w_x, w_assign, w_codes, w_codes_p, w_t1, w_dest, w_shift;  // the batch an append stores
  DeviceBuffer w_q, w_scores, w_probes, w_bits, w_refs, w_dist, w_bytes, w_key, w_order, w_lut, w_cand;
  DeviceBuffer w_pkeys, w_pcnt, w_pdone;  // sliced queries of the streaming scan
  DeviceBuffer w_delta, w_fb;             // certificate bounds; uncertified queries (count, list)
  // A filtered search's admitted codes as a store of their own: per-list counts, offsets, the
  // original position of each, and their codes, t1 terms and stored vectors.
  DeviceBuffer w_fcnt, w_foff, w_fpos, w_fcodes, w_ft1, w_fvec;
  bool last_certified = false;            // the last search ranked approximately (w_fb holds its count)
  int cus = 0;                             // compute units of the device
  int timing = 0;               // 0 off, 1 stage events, 2 events and probed code bytes
  bool timed = false, timed_bytes = false;
  hipEvent_t ev[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
  hipEvent_t join = nullptr;  // orders calls on other streams into the handle's stream
};

namespace {

__global__ void zero_u32_kernel(uint32_t* p, uint64_t n) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

int ivf_mode(const qvh_ivfpq* h) {
  if (h->metric != QVH_METRIC_L2) return kModeIp;
  return h->has_pre ? kModePre : kModeResidual;
}

/// Cells (src/ivfpq_index.cc:238) and codes (:239-245) of n device-resident rows `d_x` (already
/// normalized for cosine), into the encode workspace `es` (its assign and codes buffers). The caller
/// holds es.mu; `s` is the stream the work goes on.
void ivf_encode_device(const qvh_ivfpq* h, EncodeSpace& es, const float* d_x, uint64_t n, hipStream_t s) {
  uint32_t* assign = static_cast<uint32_t*>(es.assign.reserve(n * sizeof(uint32_t)));
  NearestArgs na{};
  na.x = d_x;
  na.n = n;
  na.dim = h->dim;
  na.x_stride = h->dim;
  na.x_off = 0;
  na.ct = h->cent_t.as<float>();
  na.norms = h->cent_norm.as<float>();
  na.k = h->nlist;
  na.max_ip = h->metric == QVH_METRIC_IP;
  na.out32 = assign;
  launch_assign(na, h->asg, es.afb, s);
  float* res = static_cast<float*>(es.res.reserve(n * h->dim * sizeof(float)));
  hipLaunchKernelGGL(residual_kernel, dim3(static_cast<unsigned>(ceil_div(n * h->dim, 256))), dim3(256), 0, s,
                     d_x, assign, h->cent.as<float>(), n, h->dim, res);
  uint8_t* codes = static_cast<uint8_t*>(es.codes.reserve(n * h->m));
  NearestArgs pa{};
  pa.x = res;
  pa.n = n;
  pa.dim = h->dsub;  // per sub-space
  pa.x_stride = h->dim;
  pa.x_off = 0;
  pa.ct = h->cbt.as<float>();
  pa.k = 256;
  pa.out8 = codes;
  pa.out_stride = h->m;
  launch_nearest(true, pa, h->m, s);
  QVH_HIP(hipGetLastError());
}

void ivf_check_trained(const qvh_ivfpq* h) {
  if (!h->trained) throw Failure(QVH_EINVAL, "IVF-PQ index must be trained before add()");
}

/// Admitted positions of list l (bit p % 64 of word p / 64 of the position bitmap), counted by one
/// wave per list.
__global__ void __launch_bounds__(256) filter_count_kernel(const uint64_t* __restrict__ off, uint32_t nlist,
                                                           const uint64_t* __restrict__ bits, uint32_t* __restrict__ cnt) {
  const uint32_t l = blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (l >= nlist) return;
  uint32_t c = 0;
  for (uint64_t p = off[l] + lane; p < off[l + 1]; p += 64) c += static_cast<uint32_t>((bits[p >> 6] >> (p & 63)) & 1ull);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
  if (lane == 0) cnt[l] = c;
}

/// off_f[l] = sum of cnt[0, l) for l <= nlist (one block of 1024 threads, each a contiguous chunk).
__global__ void __launch_bounds__(1024) filter_offsets_kernel(const uint32_t* __restrict__ cnt, uint32_t nlist,
                                                              uint64_t* __restrict__ off_f) {
  __shared__ uint64_t s_sum[1024];
  const uint32_t t = threadIdx.x;
  const uint32_t chunk = (nlist + 1023) / 1024;
  const uint32_t b = min(nlist, t * chunk), e = min(nlist, b + chunk);
  uint64_t own = 0;
  for (uint32_t i = b; i < e; ++i) own += cnt[i];
  s_sum[t] = own;
  __syncthreads();
  for (uint32_t d = 1; d < 1024; d <<= 1) {  // inclusive scan
    const uint64_t v = t >= d ? s_sum[t - d] : 0;
    __syncthreads();
    s_sum[t] += v;
    __syncthreads();
  }
  uint64_t run = s_sum[t] - own;
  for (uint32_t i = b; i < e; ++i) {
    off_f[i] = run;
    run += cnt[i];
  }
  if (t == 1023) off_f[nlist] = s_sum[1023];
}

struct FilterGatherArgs {
  const uint64_t* off;     // [nlist + 1] the store's list offsets
  const uint64_t* bits;    // position bitmap
  const uint64_t* off_f;   // [nlist + 1] the admitted codes' offsets
  uint32_t nlist;
  uint32_t mw;             // code dwords (mp / 4)
  uint32_t dim;
  const uint32_t* codes;   // [count][mw]
  const float* t1;         // [count] or null
  const float* vec;        // [count][dim] or null
  uint32_t* pos;           // [admitted] original positions
  uint32_t* codes_f;       // [admitted][mw]
  float* t1_f;             // [admitted] or null
  float* vec_f;            // [admitted][dim] or null
};

/// The admitted codes of list l, in position order, into the compact store (one wave per list).
__global__ void __launch_bounds__(256) filter_gather_kernel(FilterGatherArgs g) {
  const uint32_t l = blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (l >= g.nlist) return;
  uint64_t dst = g.off_f[l];
  const uint64_t end = g.off[l + 1];
  for (uint64_t base = g.off[l]; base < end; base += 64) {
    const uint64_t p = base + static_cast<uint64_t>(lane);
    const bool in = p < end && ((g.bits[p >> 6] >> (p & 63)) & 1ull);
    const uint64_t mask = __ballot(in);
    if (in) {
      const uint64_t d = dst + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
      g.pos[d] = static_cast<uint32_t>(p);
      for (uint32_t w = 0; w < g.mw; ++w) g.codes_f[d * g.mw + w] = g.codes[p * g.mw + w];
      if (g.t1_f) g.t1_f[d] = g.t1[p];
      if (g.vec_f) {
        for (uint32_t j = 0; j < g.dim; ++j) g.vec_f[d * g.dim + j] = g.vec[p * g.dim + j];
      }
    }
    dst += static_cast<uint64_t>(__popcll(mask));
  }
}

/// Refs over the compact store ((list << 32) | rank among the list's admitted codes) back to the
/// store's ((list << 32) | offset in the list).
__global__ void filter_remap_kernel(uint64_t* __restrict__ refs, uint64_t total, const uint64_t* __restrict__ off,
                                    const uint64_t* __restrict__ off_f, const uint32_t* __restrict__ pos) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint64_t ref = refs[i];
  if (ref == QVH_EMPTY_REF) return;
  const uint64_t l = ref >> 32;
  const uint64_t orig = pos[off_f[l] + (ref & 0xFFFFFFFFull)];
  refs[i] = (l << 32) | (orig - off[l]);
}

void ivf_search_impl(qvh_ivfpq* h, const float* d_q_raw, uint64_t nq, uint32_t k, uint32_t nprobe_req,
                     uint64_t refine_factor, const uint64_t* d_bitmap, uint64_t* d_refs, float* d_dist,
                     hipStream_t s) {
  QVH_REQUIRE(nq <= 0x7FFFFFFFull, "too many queries in one call");
  const uint32_t nprobe = std::min(std::max<uint32_t>(nprobe_req, 1), h->nlist);
  // keep = min(count, sat(k * factor)) (src/ivfpq_index.cc:303-308)
  const bool refine = refine_factor > 0 && h->store_vectors;
  const uint64_t factor = refine ? refine_factor : 1;
  const uint64_t count = h->count;
  uint64_t keep = factor > count / std::max<uint64_t>(k, 1) ? count : static_cast<uint64_t>(k) * factor;
  keep = std::min(keep, count);
  const int mode = ivf_mode(h);
  // L2 with the precomputed table selects keep + max(6, keep / 2) candidates by the approximate sum
  // and re-scores them: the margin lets the keep-th exact sum fall below the last approximate one by
  // more than the rounding bound, which certifies the ranking (1M x 128, k = 10: 16 candidates
  // rather than 26 took the scan from 0.185 to 0.177 ms at nprobe 1 and from 0.965 to 0.957 ms at
  // nprobe 32, with identical results).
  uint64_t keep_sel = keep;
  if (mode == kModePre) keep_sel = std::min<uint64_t>(count, keep + std::max<uint64_t>(6, keep / 2));
  // Refine over every stored vector (k * refine_factor at or past the count): the ADC stage keeps
  // every probed candidate, so the answer is the exact top-k of the probed, admitted vectors, which
  // the block-buffer scan computes directly (src/ivfpq_index.cc:303-308,362-373).
  bool exact_all = false;
  if (keep_sel > kMaxKeepSel && refine && keep == count) {
    exact_all = true;
    keep = std::min<uint64_t>(k, count);
    keep_sel = keep;
  }
  if (keep_sel > (uint64_t{1} << 20)) {
    throw Failure(QVH_EUNSUPPORTED, "IVF-PQ search: " + std::to_string(keep_sel) +
                                        " candidates (k * refine_factor) exceed the device path's 2^20");
  }
  uint32_t cand_cap = kCandCap;
  while (cand_cap < keep_sel + kScanThreads * kScanRound) cand_cap *= 2;
  QVH_REQUIRE(h->count < 0xFFFFFFFFull, "IVF-PQ device path holds fewer than 2^32 vectors");
  if (h->timed) QVH_HIP(hipEventRecord(h->ev[0], s));
  // Prepared queries: the caller's rows as they are (L2, inner product; 16-byte aligned for the
  // table build's vector loads), or a copy normalized in place (cosine).
  const float* dq = d_q_raw;
  if (h->metric == QVH_METRIC_COSINE || reinterpret_cast<uintptr_t>(d_q_raw) % 16 != 0) {
    float* copy = static_cast<float*>(h->w_q.reserve(nq * h->dim * sizeof(float)));
    if (copy != d_q_raw) QVH_HIP(hipMemcpyAsync(copy, d_q_raw, nq * h->dim * sizeof(float), hipMemcpyDeviceToDevice, s));
    if (h->metric == QVH_METRIC_COSINE) launch_normalize_rows(copy, nq, h->dim, s);
    dq = copy;
  }
  // coarse scores + probes
  float* scores = static_cast<float*>(h->w_scores.reserve(nq * h->nlist * sizeof(float)));
  uint32_t* probes = static_cast<uint32_t*>(h->w_probes.reserve(nq * nprobe * sizeof(uint32_t)));
  // Block order of the streaming scan (queries grouped by their smallest probed list): for batches
  // of up to 64k queries and up to 32k lists (the counts fit one block's LDS).
  const bool ordered = nq > 1 && nq <= 65536 && h->nlist <= 32768 && mode != kModeResidual && h->mp <= kStreamMaxM &&
                       nprobe <= kStreamMaxProbes;
  uint32_t* min_probe = ordered ? static_cast<uint32_t*>(h->w_key.reserve(nq * sizeof(uint32_t))) : nullptr;
  const uint64_t cg_min = nprobe > 32 ? kCgMinQueriesWide : kCgMinQueries;
  const bool mfma_coarse = h->asg.ready && h->asg.dim == h->dim && nq >= cg_min && nq < 0xFFFFFFFFull &&
                           nprobe <= kCgMaxProbes && h->nlist <= kCgMaxLists;
  if (mfma_coarse) {
    const bool ip = h->metric != QVH_METRIC_L2;
    CoarseGemmArgs ga{};
    ga.Q = dq;
    ga.nq = static_cast<uint32_t>(nq);
    ga.dim = h->dim;
    ga.crow = h->asg.crow.as<float>();
    ga.aug = h->asg.aug.as<float>();
    ga.kp = h->asg.kp;
    ga.dp = h->asg.dp;
    ga.nlist = h->nlist;
    ga.ncb = static_cast<uint32_t>(ceil_div(h->nlist, kCgTileC));
    ga.nqb = static_cast<uint32_t>(ceil_div(nq, kCgTileQ));
    ga.qb_per_xcd = static_cast<uint32_t>(ceil_div(ga.nqb, 8));
    ga.g = scores;
    const dim3 grid(8u * ga.qb_per_xcd * ga.ncb);
    if (ip) {
      hipLaunchKernelGGL(coarse_gemm_kernel<false>, grid, dim3(kCgThreads), 0, s, ga);
    } else {
      hipLaunchKernelGGL(coarse_gemm_kernel<true>, grid, dim3(kCgThreads), 0, s, ga);
    }
    BandArgs ba{};
    ba.Q = dq;
    ba.nq = static_cast<uint32_t>(nq);
    ba.dim = h->dim;
    ba.cent = h->cent.as<float>();
    ba.nlist = h->nlist;
    ba.nprobe = nprobe;
    ba.rmax = h->asg.rmax.as<float>();
    ba.coef = ldexpf(4.0f * static_cast<float>(h->asg.dp + 1) + 16.0f, -24);
    ba.scores = scores;
    ba.probes = probes;
    ba.min_probe = min_probe;
    if (mode == kModePre && !exact_all && keep > 0) {
      ba.adc_bound = static_cast<float*>(h->w_delta.reserve(nq * sizeof(float)));
      ba.fb_count = static_cast<uint32_t*>(h->w_fb.reserve((nq + 1) * sizeof(uint32_t)));
      ba.cmax = h->cmax.as<float>();
      ba.pmax = h->pmax.as<float>();
      ba.m = h->m;
      ba.dsub = h->dsub;
    }
    const dim3 bgrid(static_cast<unsigned>(ceil_div(nq, 4)));
    void (*band)(BandArgs);
    if (h->nlist <= 256 * 2) {
      band = ip ? coarse_band_kernel<true, 2> : coarse_band_kernel<false, 2>;
    } else if (h->nlist <= 256 * 4) {
      band = ip ? coarse_band_kernel<true, 4> : coarse_band_kernel<false, 4>;
    } else {
      band = ip ? coarse_band_kernel<true, 8> : coarse_band_kernel<false, 8>;
    }
    hipLaunchKernelGGL(band, bgrid, dim3(256), 0, s, ba);
  } else {
    const bool single = nq <= kCoarseSingleMaxQ;
    const dim3 grid(static_cast<unsigned>(ceil_div(h->nlist, 256)),
                    static_cast<unsigned>(single ? nq : ceil_div(nq, kCoarseQ)));
    const bool ip = h->metric != QVH_METRIC_L2;
    auto kern = single ? (ip ? coarse_kernel<true, 1> : coarse_kernel<false, 1>)
                       : (ip ? coarse_kernel<true, kCoarseQ> : coarse_kernel<false, kCoarseQ>);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, dq, static_cast<uint32_t>(nq), h->dim, h->cent_t.as<float>(),
                       h->nlist, scores);
    const dim3 sgrid(static_cast<unsigned>(ceil_div(nq, 4)));
    const uint32_t nq32 = static_cast<uint32_t>(nq);
    if (h->nlist <= 64 * 8) {
      hipLaunchKernelGGL(probe_select_kernel<8>, sgrid, dim3(256), 0, s, scores, nq32, h->nlist, nprobe, probes, min_probe);
    } else if (h->nlist <= 64 * 32) {
      hipLaunchKernelGGL(probe_select_kernel<32>, sgrid, dim3(256), 0, s, scores, nq32, h->nlist, nprobe, probes, min_probe);
    } else {
      hipLaunchKernelGGL(probe_select_any_kernel, sgrid, dim3(256), 0, s, scores, nq32, h->nlist, nprobe, probes,
                         min_probe);
    }
  }
  uint32_t* order = nullptr;
  if (ordered) {
    order = static_cast<uint32_t*>(h->w_order.reserve(nq * sizeof(uint32_t)));
    const size_t olds = static_cast<size_t>(h->nlist) * sizeof(uint32_t);
    if (olds > 64 * 1024) {
      QVH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(probe_order_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(olds)));
    }
    hipLaunchKernelGGL(probe_order_kernel, dim3(1), dim3(1024), olds, s, min_probe, static_cast<uint32_t>(nq), h->nlist,
                       order);
  }
  // L2 with the precomputed table ranks candidates by an approximate sum and re-scores the best:
  // each query's bound on the rounding difference certifies the ranking (adc_bound_kernel), and the
  // queries it does not certify are listed in fb for an exact rescan.
  const bool certify = mode == kModePre && !exact_all && keep > 0;
  float* delta = nullptr;
  uint32_t* fb = nullptr;
  if (certify) {
    delta = static_cast<float*>(h->w_delta.reserve(nq * sizeof(float)));
    fb = static_cast<uint32_t*>(h->w_fb.reserve((nq + 1) * sizeof(uint32_t)));
  }
  if (certify && !mfma_coarse) {  // the band kernel computes the bound itself
    hipLaunchKernelGGL(adc_bound_kernel, dim3(static_cast<unsigned>(ceil_div(nq, 4))), dim3(256), 0, s, dq,
                       static_cast<uint32_t>(nq), h->dim, h->m, h->dsub, h->cmax.as<float>(), scores, h->nlist, probes,
                       nprobe, h->pmax.as<float>(), delta, fb);
  }
  h->last_certified = certify;
  QVH_HIP(hipGetLastError());
  // A filter: the admitted codes (and t1 terms and stored vectors) become a store of their own,
  // which the scans read like an unfiltered one, so their work follows the admitted count as the
  // reference's skip of filtered labels does (src/ivfpq_index.cc:349); the refs they write are
  // mapped back to the store's afterwards. Buffers are sized for every stored code (no count read
  // back), and grow once.
  const uint64_t* off_use = h->off.as<uint64_t>();
  const uint8_t* codes_use = h->codes.as<uint8_t>();
  const float* t1_use = h->t1.as<float>();
  const float* vec_use = h->vec.as<float>();
  uint64_t* off_f = nullptr;
  uint32_t* fpos = nullptr;
  if (d_bitmap != nullptr && count > 0) {
    const uint32_t nl = h->nlist;
    uint32_t* fcnt = static_cast<uint32_t*>(h->w_fcnt.reserve(nl * sizeof(uint32_t)));
    off_f = static_cast<uint64_t*>(h->w_foff.reserve((nl + 1) * sizeof(uint64_t)));
    fpos = static_cast<uint32_t*>(h->w_fpos.reserve(count * sizeof(uint32_t)));
    FilterGatherArgs g{};
    g.off = off_use;
    g.bits = d_bitmap;
    g.off_f = off_f;
    g.nlist = nl;
    g.mw = h->mp / 4;
    g.dim = h->dim;
    g.codes = reinterpret_cast<const uint32_t*>(codes_use);
    g.t1 = h->has_pre ? t1_use : nullptr;
    g.vec = h->store_vectors ? vec_use : nullptr;
    g.pos = fpos;
    g.codes_f = static_cast<uint32_t*>(h->w_fcodes.reserve(count * h->mp));
    g.t1_f = g.t1 ? static_cast<float*>(h->w_ft1.reserve(count * sizeof(float))) : nullptr;
    g.vec_f = g.vec ? static_cast<float*>(h->w_fvec.reserve(count * h->dim * sizeof(float))) : nullptr;
    const dim3 wave_grid(static_cast<unsigned>(ceil_div(nl, 4)));
    hipLaunchKernelGGL(filter_count_kernel, wave_grid, dim3(256), 0, s, off_use, nl, d_bitmap, fcnt);
    hipLaunchKernelGGL(filter_offsets_kernel, dim3(1), dim3(1024), 0, s, fcnt, nl, off_f);
    hipLaunchKernelGGL(filter_gather_kernel, wave_grid, dim3(256), 0, s, g);
    QVH_HIP(hipGetLastError());
    off_use = off_f;
    codes_use = reinterpret_cast<const uint8_t*>(g.codes_f);
    t1_use = g.t1_f;
    vec_use = g.vec_f;
  }
  if (h->timed) QVH_HIP(hipEventRecord(h->ev[1], s));
  ScanArgs a{};
  a.delta = delta;
  a.fallback = fb ? fb + 1 : nullptr;
  a.nfallback = fb;
  a.nq = static_cast<uint32_t>(nq);
  a.k = k;
  a.m = h->m;
  a.mp = h->mp;
  a.dsub = h->dsub;
  a.dim = h->dim;
  a.nlist = h->nlist;
  a.nprobe = nprobe;
  a.mode = mode;
  a.Q = dq;
  a.scores = scores;
  a.probes = probes;
  a.off = off_use;
  a.codes = codes_use;
  a.t1 = t1_use;
  a.pre = h->pre.as<float>();
  a.cbt = h->cbt.as<float>();
  a.cbc = h->cbc.as<float>();
  a.cent = h->cent.as<float>();
  a.vec = vec_use;
  a.bitmap = off_f != nullptr ? nullptr : d_bitmap;
  a.keep = static_cast<uint32_t>(keep);
  a.keep_sel = static_cast<uint32_t>(keep_sel);
  a.refine = refine && !exact_all ? 1 : 0;
  a.exact_all = exact_all ? 1 : 0;
  a.out_refs = d_refs;
  a.out_dist = d_dist;
  a.cand_cap = cand_cap;
  // m above kScanMaxLdsM: the block-buffer scan's tables in global memory, one per work-group, and
  // a bounded grid whose work-groups take the queries in turn.
  const bool table_global = h->m > kScanMaxLdsM;
  const size_t table_bytes = static_cast<size_t>(h->m) * 256 * sizeof(float);
  // A candidate buffer that does not fit LDS beside the rest moves to global memory the same way.
  const size_t cand_bytes = static_cast<size_t>(cand_cap) * sizeof(uint64_t);
  const size_t lds_rest =
      (nprobe + 1) * sizeof(uint64_t) + ((nprobe + 1) & ~1u) * sizeof(uint32_t) + (table_global ? 0 : table_bytes);
  const bool cand_global = cand_bytes + lds_rest > kScanMaxLds;
  const uint64_t block_grid = std::max<uint64_t>(
      1, std::min<uint64_t>({nq, 2 * static_cast<uint64_t>(std::max(h->cus, 1)), kScanGlobalTableBytes / table_bytes,
                             cand_global ? kScanGlobalCandBytes / cand_bytes : nq}));
  const size_t lds = (cand_global ? 0 : cand_bytes) + lds_rest;
  if (lds > kScanMaxLds) {
    throw Failure(QVH_EUNSUPPORTED, "IVF-PQ search: nprobe = " + std::to_string(nprobe) +
                                        " probed lists exceed the block-buffer scan's on-chip list table");
  }
  if (table_global) a.lut_global = static_cast<float*>(h->w_lut.reserve(block_grid * table_bytes));
  if (cand_global) a.cand_global = static_cast<uint64_t*>(h->w_cand.reserve(block_grid * cand_bytes));
  const bool bounded_grid = table_global || cand_global;
  const dim3 grid(static_cast<unsigned>(bounded_grid ? block_grid : nq));
  const uint32_t mpw = h->mp / 4;
  // The block-buffer scan (every table mode, any candidate count up to kMaxKeepSel).
  auto launch_block_scan = [&](const ScanArgs& args, dim3 g) {
    auto go = [&](auto kernel) {
      const void* fn = reinterpret_cast<const void*>(kernel);
      if (lds > 64 * 1024) {
        QVH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
      }
      hipLaunchKernelGGL(kernel, g, dim3(kScanThreads), lds, s, args);
    };
    if (mpw <= 2) {
      go(ivf_scan_kernel<2>);
    } else if (mpw <= 4) {
      go(ivf_scan_kernel<4>);
    } else if (mpw <= 8) {
      go(ivf_scan_kernel<8>);
    } else if (mpw <= 16) {
      go(ivf_scan_kernel<16>);
    } else {
      go(ivf_scan_kernel<32>);  // 128 sub-spaces per pass over a code
    }
  };
  if (keep == 0) {
    // nothing stored: every slot is empty
    a.keep_sel = 0;
  }
  // Dynamic LDS above the default 64 KiB needs the kernel's limit raised first.
  auto raise_lds = [&](const void* fn, size_t bytes) {
    if (bytes > 64 * 1024) {
      QVH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
    }
  };
  // The streaming scan covers the table modes with up to 256 probes, m <= 64 and a candidate set of
  // at most 256; the rest takes the block-buffer scan below.
  const uint32_t mpw_t = mpw <= 8 ? mpw : 16;  // the kernel's code width in dwords
  const bool full = h->mp == 4 * mpw_t;
  const bool small_sel = a.keep_sel <= 64 && k <= 64;
  const bool big_sel = !small_sel && (a.keep_sel > 128 || k > 128);  // 512-entry wave queues
  // 1024-entry wave queues for 257..512 candidates (codes of up to 32 bytes; wider codes take the
  // block-buffer scan). 1M x 128 L2, nprobe 32, 10k queries, k = 200 (300 candidates): 8.80 ms on
  // the block-buffer scan.
  const bool huge_sel = a.keep_sel > 256 || k > 256;
  // Four-wave blocks take 192-entry queues past 48 candidates, so that at least 64 candidates
  // arrive between two cuts of a queue (1M x 128, nprobe 16: 60 candidates 0.97 -> 0.84 ms; at 36-40
  // candidates the 128-entry queues measured 1-2% faster).
  const bool mid_sel = small_sel && a.keep_sel > 48;
  const uint32_t cap = small_sel ? (mid_sel ? 192 : 128) : huge_sel ? 1024 : big_sel ? 512 : 256;
  // 256-entry queues run on four waves, except for L2 with the precomputed table, whose block
  // re-scores its selection: 1.18M x 100 cosine, refine 8 (80 candidates), nprobe 16 0.69 ->
  // 0.66 ms and nprobe 64 1.86 -> 1.81 ms on four waves; 1M x 128 L2, k = 50 (75 candidates),
  // nprobe 32 1.16 -> 1.25 ms.
  const bool four256 = cap == 256 && mode != kModePre;
  const size_t rows = 4 * mpw_t;
  // LDS of the streaming kernels: the table (static LDS for codes of up to 32 bytes), the wave
  // queues and the probed-list arrays (dynamic).
  const size_t lds_table = rows * 256 * sizeof(float);
  const uint32_t waves = small_sel || four256 ? 4u : 8u;
  const size_t lds_total = lds_table + static_cast<size_t>(waves) * cap * sizeof(uint64_t) +
                           (4 * static_cast<size_t>(nprobe) + 2 + waves) * sizeof(uint32_t);
  const size_t lds2 = mpw_t > 8 ? lds_total : lds_total - lds_table;
  if (!exact_all && mode != kModeResidual && h->mp <= kStreamMaxM && nprobe <= kStreamMaxProbes && a.keep_sel >= 1 &&
      a.keep_sel <= kStreamMaxSel && k <= kStreamMaxSel && !(huge_sel && mpw_t > 8) && lds_total <= 150 * 1024) {
    a.order = order;
    auto launch2 = [&](auto kernel) {
      const void* fn = reinterpret_cast<const void*>(kernel);
      raise_lds(fn, lds2);
      // Sliced queries: a batch smaller than one resident generation of blocks would leave CUs
      // idle, so each of its queries is scanned in up to kMaxSlices slices (as many as fit in one
      // generation), merged by the slice that finishes last. Larger batches scan whole queries:
      // slicing their last generation measured no faster at 10k queries and slower at 2k.
      int per_cu = 0;
      QVH_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, static_cast<int>(waves * 64), lds2));
      const uint64_t resident = static_cast<uint64_t>(std::max(per_cu, 0)) * static_cast<uint64_t>(std::max(h->cus, 0));
      uint64_t parts = resident > nq ? std::min<uint64_t>(kMaxSlices, resident / nq) : 1;
      uint64_t sliced = nq;
      // The merging block holds parts * keep keys: in one wave's registers (256) or in the queues.
      const uint64_t cap_keys = small_sel ? 256u : static_cast<uint64_t>(waves) * cap;
      while (parts > 1 && parts * a.keep > cap_keys) --parts;
      if (parts <= 1 || a.keep == 0) sliced = 0;
      a.nwhole = static_cast<uint32_t>(nq - sliced);
      a.parts = sliced ? static_cast<uint32_t>(parts) : 1u;
      if (sliced) {
        a.part_keys = static_cast<uint64_t*>(h->w_pkeys.reserve(sliced * parts * a.keep * sizeof(uint64_t)));
        a.part_cnt = static_cast<uint32_t*>(h->w_pcnt.reserve(sliced * parts * sizeof(uint32_t)));
        const size_t had = h->w_pdone.bytes;
        a.part_done = static_cast<uint32_t*>(h->w_pdone.reserve(sliced * sizeof(uint32_t)));
        if (h->w_pdone.bytes != had) {  // fresh counters start at zero; the merging block resets them
          const uint64_t n = h->w_pdone.bytes / sizeof(uint32_t);
          hipLaunchKernelGGL(zero_u32_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s, a.part_done, n);
        }
      }
      const dim3 sgrid(static_cast<unsigned>(a.nwhole + sliced * a.parts));
      hipLaunchKernelGGL(kernel, sgrid, dim3(waves * 64), lds2, s, a);
    };
#define QVH_STREAM_CAP(KERNEL, ...)                                                                       \
  (small_sel ? (mid_sel ? launch2(KERNEL<__VA_ARGS__, 192>) : launch2(KERNEL<__VA_ARGS__, 128>))          \
   : big_sel ? launch2(KERNEL<__VA_ARGS__, 512>)                                                          \
   : four256 ? launch2(KERNEL<__VA_ARGS__, 256, false, 4>) : launch2(KERNEL<__VA_ARGS__, 256>))
#define QVH_STREAM(MPW_)                                                                                  \
  (huge_sel ? launch2(ivf_stream_kernel<MPW_, true, 1024>) : QVH_STREAM_CAP(ivf_stream_kernel, MPW_, true))
    // Bank-rotated lookups: L2 with the precomputed table (re-scored exactly afterwards), four
    // dims per sub-space, 16- or 32-byte codes.
    const bool rot =
        QVH_STREAM_ROT && mode == kModePre && full && h->dsub == 4 && (mpw_t == 4 || mpw_t == 8) && !big_sel && !mid_sel;
    if (rot && mpw_t == 8) {
      small_sel ? launch2(ivf_stream_kernel<8, true, 128, true>) : launch2(ivf_stream_kernel<8, true, 256, true>);
    } else if (rot) {
      small_sel ? launch2(ivf_stream_kernel<4, true, 128, true>) : launch2(ivf_stream_kernel<4, true, 256, true>);
    } else if (mpw_t == 1) {
      QVH_STREAM(1);
    } else if (mpw_t == 2) {
      QVH_STREAM(2);
    } else if (mpw_t == 3) {
      QVH_STREAM(3);
    } else if (mpw_t == 4) {
      QVH_STREAM(4);
    } else if (mpw_t == 5) {
      QVH_STREAM(5);
    } else if (mpw_t == 6) {
      QVH_STREAM(6);
    } else if (mpw_t == 7) {
      QVH_STREAM(7);
    } else if (mpw_t == 8) {
      QVH_STREAM(8);
    } else if (full) {
      QVH_STREAM_CAP(ivf_stream_wide_kernel, true);
    } else {
      QVH_STREAM_CAP(ivf_stream_wide_kernel, false);
    }
#undef QVH_STREAM
#undef QVH_STREAM_CAP
    QVH_HIP(hipGetLastError());
  } else {
    launch_block_scan(a, grid);
  }
  QVH_HIP(hipGetLastError());
  // The scan stage ends here; the rescan of uncertified queries (normally an empty launch) follows.
  if (h->timed) QVH_HIP(hipEventRecord(h->ev[2], s));
  if (certify) {
    // Exact rescan of the uncertified queries (normally none): the block-buffer scan with the
    // reference's sum for every code, over the listed queries, after every kernel above.
    ScanArgs fa = a;
    fa.exact_pre = 1;
    fa.keep_sel = fa.keep;
    fa.qlist = fb + 1;
    fa.qcount = fb;
    launch_block_scan(fa, dim3(static_cast<unsigned>(bounded_grid ? block_grid
                                                                  : std::min<uint64_t>(nq, 2 * static_cast<uint64_t>(std::max(h->cus, 1))))));
    QVH_HIP(hipGetLastError());
  }
  if (off_f != nullptr) {
    hipLaunchKernelGGL(filter_remap_kernel, dim3(static_cast<unsigned>(ceil_div(nq * k, 256))), dim3(256), 0, s, d_refs,
                       nq * k, h->off.as<uint64_t>(), off_f, fpos);
    QVH_HIP(hipGetLastError());
  }
  if (h->timed_bytes) {
    uint64_t* bytes = static_cast<uint64_t*>(h->w_bytes.reserve(sizeof(uint64_t)));
    hipLaunchKernelGGL(probed_code_bytes_kernel, dim3(1), dim3(256), 0, s, probes, nq * nprobe, a.off, h->m, bytes);
    QVH_HIP(hipGetLastError());
  }
}

}  // namespace

extern "C" {

qvh_status qvh_ivfpq_create(uint32_t dim, int metric, uint32_t nlist, uint32_t m, int store_vectors,
                            qvh_ivfpq** out) {
  return guarded([&] {
    QVH_REQUIRE(out != nullptr, "qvh_ivfpq_create: null output");
    *out = nullptr;
    QVH_REQUIRE(dim >= 1 && dim <= 65536, "dimension must be in [1, 65536]");
    QVH_REQUIRE(metric >= QVH_METRIC_L2 && metric <= QVH_METRIC_COSINE, "unknown metric");
    QVH_REQUIRE(nlist >= 1 && nlist <= (1u << 24), "nlist must be in [1, 2^24]");
    QVH_REQUIRE(m >= 1 && dim % m == 0, "PQ: dimension must be divisible by m");

    const int dev = current_device();
    auto* h = new qvh_ivfpq;
    h->dim = dim;
    h->metric = metric;
    h->nlist = nlist;
    h->m = m;
    h->dsub = dim / m;
    h->mp = (m + 3) / 4 * 4;
    h->store_vectors = store_vectors;
    h->device = dev;
    if (hipDeviceGetAttribute(&h->cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) h->cus = 0;
    h->h_off.assign(nlist + 1, 0);
    hipError_t e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e == hipSuccess) {
      e = hipStreamCreateWithFlags(&h->enc.stream, hipStreamNonBlocking);
      if (e != hipSuccess) (void)hipStreamDestroy(h->stream);
    }
    if (e != hipSuccess) {
      delete h;
      throw Failure(QVH_EDEVICE, std::string("hipStreamCreate: ") + hipGetErrorString(e));
    }
    try {
      h->off.reserve((nlist + 1) * sizeof(uint64_t));
      QVH_HIP(hipMemcpy(h->off.ptr, h->h_off.data(), (nlist + 1) * sizeof(uint64_t), hipMemcpyHostToDevice));
    } catch (...) {
      (void)hipStreamDestroy(h->stream);
      (void)hipStreamDestroy(h->enc.stream);
      delete h;
      throw;
    }
    *out = h;
  });
}

void qvh_ivfpq_destroy(qvh_ivfpq* h) {
  if (!h) return;
  (void)hipSetDevice(h->device);
  if (h->stream) {
    (void)hipStreamSynchronize(h->stream);
    (void)hipStreamDestroy(h->stream);
  }
  if (h->enc.stream) {
    (void)hipStreamSynchronize(h->enc.stream);
    (void)hipStreamDestroy(h->enc.stream);
  }
  for (hipEvent_t& e : h->ev) {
    if (e) (void)hipEventDestroy(e);
  }
  if (h->join) (void)hipEventDestroy(h->join);
  delete h;
}

qvh_status qvh_ivfpq_set_trained(qvh_ivfpq* h, const float* centroids, const float* codebook,
                                 int use_precomputed) {
  return guarded([&] {
    QVH_REQUIRE(h && centroids && codebook, "qvh_ivfpq_set_trained: null argument");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_REQUIRE(!h->trained, "index is already trained");
    QVH_HIP(hipSetDevice(h->device));
    hipStream_t s = h->stream;
    const uint64_t cbytes = static_cast<uint64_t>(h->nlist) * h->dim * sizeof(float);
    const uint64_t bbytes = static_cast<uint64_t>(h->m) * 256 * h->dsub * sizeof(float);
    h->cent.reserve(cbytes);
    h->cent_t.reserve(cbytes);
    h->cent_norm.reserve(h->nlist * sizeof(float));
    h->cb.reserve(bbytes);
    h->cbt.reserve(bbytes);
    h->cbc.reserve(bbytes);
    QVH_HIP(hipMemcpyAsync(h->cent.ptr, centroids, cbytes, hipMemcpyHostToDevice, s));
    QVH_HIP(hipMemcpyAsync(h->cb.ptr, codebook, bbytes, hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(centroid_prep_kernel, dim3(static_cast<unsigned>(ceil_div(h->nlist, 256))), dim3(256), 0, s,
                       h->cent.as<float>(), h->nlist, h->dim, h->cent_t.as<float>(), h->cent_norm.as<float>());
    prepare_assign_table(h->asg, h->cent.as<float>(), h->cent_norm.as<float>(), h->nlist, h->dim,
                         h->metric == QVH_METRIC_IP, s);
    hipLaunchKernelGGL(codebook_prep_kernel, dim3(static_cast<unsigned>(ceil_div(uint64_t(h->m) * 256 * h->dsub, 256))),
                       dim3(256), 0, s, h->cb.as<float>(), h->m, h->dsub, h->cbt.as<float>());
    hipLaunchKernelGGL(codebook_cmajor_kernel, dim3(static_cast<unsigned>(ceil_div(uint64_t(h->m) * 256 * h->dsub, 256))),
                       dim3(256), 0, s, h->cb.as<float>(), h->m, h->dsub, h->cbc.as<float>());
    h->has_pre = use_precomputed != 0 && h->metric == QVH_METRIC_L2;
    if (h->has_pre) {
      const uint64_t n = static_cast<uint64_t>(h->nlist) * h->m * 256;
      h->pre.reserve(n * sizeof(float));
      hipLaunchKernelGGL(precompute_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s,
                         h->cent.as<float>(), h->cb.as<float>(), h->nlist, h->dim, h->m, h->pre.as<float>());
      h->pmax.reserve(h->nlist * sizeof(float));
      hipLaunchKernelGGL(pre_bound_kernel, dim3(h->nlist), dim3(256), 0, s, h->pre.as<float>(), h->m,
                         h->pmax.as<float>());
      h->cmax.reserve(h->m * sizeof(float));
      hipLaunchKernelGGL(codeword_norm_kernel, dim3(static_cast<unsigned>(ceil_div(h->m, 64))), dim3(64), 0, s,
                         h->cb.as<float>(), h->m, h->dsub, h->cmax.as<float>());
    }
    QVH_HIP(hipGetLastError());
    QVH_HIP(hipStreamSynchronize(s));
    h->trained.store(true, std::memory_order_release);
  });
}

qvh_status qvh_ivfpq_precomputed(qvh_ivfpq* h, float* out) {
  return guarded([&] {
    QVH_REQUIRE(h && out, "qvh_ivfpq_precomputed: null argument");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_REQUIRE(h->has_pre, "no precomputed table (metric is not L2 or it exceeds the budget)");
    QVH_HIP(hipSetDevice(h->device));
    QVH_HIP(hipMemcpy(out, h->pre.ptr, static_cast<uint64_t>(h->nlist) * h->m * 256 * sizeof(float),
                      hipMemcpyDeviceToHost));
  });
}

qvh_status qvh_ivfpq_encode(qvh_ivfpq* h, const float* x, uint64_t n, uint32_t* assign, uint8_t* codes,
                            float* stored_out) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_encode: null handle");
    if (n == 0) return;
    QVH_REQUIRE(x != nullptr, "qvh_ivfpq_encode: null vectors");
    EncodeSpace& es = h->enc;
    std::lock_guard<std::mutex> lock(es.mu);  // not the handle's lock: searches go on meanwhile
    QVH_REQUIRE(h->trained.load(std::memory_order_acquire), "IVF-PQ index must be trained before add()");
    QVH_HIP(hipSetDevice(h->device));
    hipStream_t s = es.stream;
    float* dx = static_cast<float*>(es.x.reserve(n * h->dim * sizeof(float)));
    QVH_HIP(hipMemcpyAsync(dx, x, n * h->dim * sizeof(float), hipMemcpyHostToDevice, s));
    if (h->metric == QVH_METRIC_COSINE) launch_normalize_rows(dx, n, h->dim, s);
    ivf_encode_device(h, es, dx, n, s);
    if (assign) QVH_HIP(hipMemcpyAsync(assign, es.assign.ptr, n * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    if (codes) QVH_HIP(hipMemcpyAsync(codes, es.codes.ptr, n * h->m, hipMemcpyDeviceToHost, s));
    if (stored_out) QVH_HIP(hipMemcpyAsync(stored_out, dx, n * h->dim * sizeof(float), hipMemcpyDeviceToHost, s));
    QVH_HIP(hipStreamSynchronize(s));
  });
}

namespace {

/// Appends n encoded entries to the lists, each after its list's existing entries in batch order
/// (src/ivfpq_index.cc:250-269): cells d_assign / h_assign (device and host copies), codes d_codes
/// [n][m], and with stored vectors d_vec [n][dim]. Builds the new CSR arrays on stream s and swaps
/// them in once s is done. The caller holds the handle's lock.
void ivf_append(qvh_ivfpq* h, const uint32_t* h_assign, const uint32_t* d_assign, const uint8_t* d_codes,
                const float* d_vec, uint64_t n, hipStream_t s) {
  const uint32_t nl = h->nlist;
  std::vector<uint64_t> add(nl, 0);
  for (uint64_t i = 0; i < n; ++i) {
    QVH_REQUIRE(h_assign[i] < nl, "qvh_ivfpq_append: cell out of range");
    ++add[h_assign[i]];
  }
  for (uint32_t l = 0; l < nl; ++l) {
    QVH_REQUIRE(h->h_off[l + 1] - h->h_off[l] + add[l] <= 0xFFFFFFFFull,
                "too many vectors in one IVF cell (2^32 limit); use a larger nlist");
  }
  const uint64_t total = h->count + n;
  QVH_REQUIRE(total < 0xFFFFFFFFull, "IVF-PQ device path holds fewer than 2^32 vectors");
  std::vector<uint64_t> shift(nl, 0), new_off(nl + 1, 0), cursor(nl, 0);
  for (uint32_t l = 0; l < nl; ++l) {
    shift[l] = l ? shift[l - 1] + add[l - 1] : 0;
    new_off[l + 1] = new_off[l] + (h->h_off[l + 1] - h->h_off[l]) + add[l];
    cursor[l] = new_off[l] + (h->h_off[l + 1] - h->h_off[l]);
  }
  std::vector<uint64_t> dest(n);
  for (uint64_t i = 0; i < n; ++i) dest[i] = cursor[h_assign[i]]++;
  // padded codes and term1 of the batch
  uint8_t* cp = static_cast<uint8_t*>(h->w_codes_p.reserve(n * h->mp));
  hipLaunchKernelGGL(pad_codes_kernel, dim3(static_cast<unsigned>(ceil_div(n * h->mp, 256))), dim3(256), 0, s,
                     d_codes, h->m, h->mp, n, cp);
  float* nt1 = nullptr;
  if (h->has_pre) {
    nt1 = static_cast<float*>(h->w_t1.reserve(n * sizeof(float)));
    hipLaunchKernelGGL(term1_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s,
                       cp, h->mp, d_assign, h->pre.as<float>(), h->m, n, nt1);
  }
  uint64_t* ddest = static_cast<uint64_t*>(h->w_dest.reserve(n * sizeof(uint64_t)));
  uint64_t* dshift = static_cast<uint64_t*>(h->w_shift.reserve(nl * sizeof(uint64_t)));
  QVH_HIP(hipMemcpyAsync(ddest, dest.data(), n * sizeof(uint64_t), hipMemcpyHostToDevice, s));
  QVH_HIP(hipMemcpyAsync(dshift, shift.data(), nl * sizeof(uint64_t), hipMemcpyHostToDevice, s));
  // new CSR buffers
  DeviceBuffer ncodes, nt1buf, nvec, noff;
  ncodes.reserve(total * h->mp);
  if (h->has_pre) nt1buf.reserve(total * sizeof(float));
  if (h->store_vectors) nvec.reserve(total * h->dim * sizeof(float));
  noff.reserve((nl + 1) * sizeof(uint64_t));
  QVH_HIP(hipMemcpyAsync(noff.ptr, new_off.data(), (nl + 1) * sizeof(uint64_t), hipMemcpyHostToDevice, s));
  ScatterArgs sa{};
  sa.old_off = h->off.as<uint64_t>();
  sa.shift = dshift;
  sa.nlist = nl;
  sa.old_count = h->count;
  sa.n_new = n;
  sa.dest = ddest;
  sa.mp = h->mp;
  sa.dim = h->dim;
  sa.old_codes = h->codes.as<uint8_t>();
  sa.new_codes = cp;
  sa.codes = ncodes.as<uint8_t>();
  sa.old_t1 = h->t1.as<float>();
  sa.new_t1 = nt1;
  sa.t1 = h->has_pre ? nt1buf.as<float>() : nullptr;
  sa.old_vec = h->vec.as<float>();
  sa.new_vec = d_vec;
  sa.vec = h->store_vectors ? nvec.as<float>() : nullptr;
  if (h->count) {
    hipLaunchKernelGGL(scatter_old_kernel, dim3(static_cast<unsigned>(ceil_div(h->count, 256))), dim3(256), 0, s, sa);
  }
  hipLaunchKernelGGL(scatter_new_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s, sa);
  QVH_HIP(hipGetLastError());
  QVH_HIP(hipStreamSynchronize(s));
  std::swap(h->codes.ptr, ncodes.ptr);
  std::swap(h->codes.bytes, ncodes.bytes);
  std::swap(h->t1.ptr, nt1buf.ptr);
  std::swap(h->t1.bytes, nt1buf.bytes);
  std::swap(h->vec.ptr, nvec.ptr);
  std::swap(h->vec.bytes, nvec.bytes);
  std::swap(h->off.ptr, noff.ptr);
  std::swap(h->off.bytes, noff.bytes);
  h->h_off = std::move(new_off);
  h->count = total;
}

}  // namespace

qvh_status qvh_ivfpq_append(qvh_ivfpq* h, const uint32_t* assign, const uint8_t* codes, const float* vectors,
                            uint64_t n) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_append: null handle");
    if (n == 0) return;
    QVH_REQUIRE(assign != nullptr && codes != nullptr, "qvh_ivfpq_append: null cells or codes");
    QVH_REQUIRE(!h->store_vectors || vectors != nullptr, "qvh_ivfpq_append: the index stores vectors: pass them");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_REQUIRE(h->trained.load(std::memory_order_acquire), "IVF-PQ index must be trained before add()");
    QVH_HIP(hipSetDevice(h->device));
    hipStream_t s = h->stream;
    uint32_t* da = static_cast<uint32_t*>(h->w_assign.reserve(n * sizeof(uint32_t)));
    uint8_t* dc = static_cast<uint8_t*>(h->w_codes.reserve(n * h->m));
    QVH_HIP(hipMemcpyAsync(da, assign, n * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    QVH_HIP(hipMemcpyAsync(dc, codes, n * h->m, hipMemcpyHostToDevice, s));
    float* dv = nullptr;
    if (h->store_vectors) {
      dv = static_cast<float*>(h->w_x.reserve(n * h->dim * sizeof(float)));
      QVH_HIP(hipMemcpyAsync(dv, vectors, n * h->dim * sizeof(float), hipMemcpyHostToDevice, s));
    }
    ivf_append(h, assign, da, dc, dv, n, s);
  });
}

qvh_status qvh_ivfpq_add(qvh_ivfpq* h, const float* x, uint64_t n, uint32_t* assign_out) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_add: null handle");
    if (n == 0) return;
    QVH_REQUIRE(x != nullptr, "qvh_ivfpq_add: null vectors");
    std::lock_guard<std::mutex> lock(h->mu);
    EncodeSpace& es = h->enc;
    std::lock_guard<std::mutex> enc_lock(es.mu);  // always after the handle's lock
    QVH_REQUIRE(h->trained.load(std::memory_order_acquire), "IVF-PQ index must be trained before add()");
    QVH_HIP(hipSetDevice(h->device));
    hipStream_t s = h->stream;
    float* dx = static_cast<float*>(es.x.reserve(n * h->dim * sizeof(float)));
    QVH_HIP(hipMemcpyAsync(dx, x, n * h->dim * sizeof(float), hipMemcpyHostToDevice, s));
    if (h->metric == QVH_METRIC_COSINE) launch_normalize_rows(dx, n, h->dim, s);
    ivf_encode_device(h, es, dx, n, s);
    std::vector<uint32_t> assign(n);
    QVH_HIP(hipMemcpyAsync(assign.data(), es.assign.ptr, n * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    QVH_HIP(hipStreamSynchronize(s));
    ivf_append(h, assign.data(), es.assign.as<uint32_t>(), es.codes.as<uint8_t>(), dx, n, s);
    if (assign_out) std::memcpy(assign_out, assign.data(), n * sizeof(uint32_t));
  });
}

qvh_status qvh_ivfpq_set_lists(qvh_ivfpq* h, const uint64_t* offsets, const uint8_t* codes,
                               const float* vectors) {
  return guarded([&] {
    QVH_REQUIRE(h && offsets, "qvh_ivfpq_set_lists: null argument");
    std::lock_guard<std::mutex> lock(h->mu);
    ivf_check_trained(h);
    QVH_REQUIRE(h->count == 0, "qvh_ivfpq_set_lists: the index already holds vectors");
    const uint32_t nl = h->nlist;
    QVH_REQUIRE(offsets[0] == 0, "list offsets must start at 0");
    for (uint32_t l = 0; l < nl; ++l) {
      QVH_REQUIRE(offsets[l] <= offsets[l + 1], "list offsets must not decrease");
      QVH_REQUIRE(offsets[l + 1] - offsets[l] <= 0xFFFFFFFFull, "too many vectors in one IVF cell");
    }
    const uint64_t count = offsets[nl];
    if (count == 0) return;
    QVH_REQUIRE(count < 0xFFFFFFFFull, "IVF-PQ device path holds fewer than 2^32 vectors");
    QVH_REQUIRE(codes != nullptr, "qvh_ivfpq_set_lists: null codes");
    QVH_REQUIRE(!h->store_vectors || vectors != nullptr, "qvh_ivfpq_set_lists: vectors are required");
    QVH_HIP(hipSetDevice(h->device));
    hipStream_t s = h->stream;
    DeviceBuffer ncodes, nt1, nvec, noff, raw, lists;
    ncodes.reserve(count * h->mp);
    noff.reserve((nl + 1) * sizeof(uint64_t));
    raw.reserve(count * h->m);
    QVH_HIP(hipMemcpyAsync(noff.ptr, offsets, (nl + 1) * sizeof(uint64_t), hipMemcpyHostToDevice, s));
    QVH_HIP(hipMemcpyAsync(raw.ptr, codes, count * h->m, hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(pad_codes_kernel, dim3(static_cast<unsigned>(ceil_div(count * h->mp, 256))), dim3(256), 0, s,
                       raw.as<uint8_t>(), h->m, h->mp, count, ncodes.as<uint8_t>());
    if (h->has_pre) {
      lists.reserve(count * sizeof(uint32_t));
      nt1.reserve(count * sizeof(float));
      hipLaunchKernelGGL(position_lists_kernel, dim3(static_cast<unsigned>(ceil_div(count, 256))), dim3(256), 0, s,
                         noff.as<uint64_t>(), nl, count, lists.as<uint32_t>());
      hipLaunchKernelGGL(term1_kernel, dim3(static_cast<unsigned>(ceil_div(count, 256))), dim3(256), 0, s,
                         ncodes.as<uint8_t>(), h->mp, lists.as<uint32_t>(), h->pre.as<float>(), h->m, count,
                         nt1.as<float>());
    }
    if (h->store_vectors) {
      nvec.reserve(count * h->dim * sizeof(float));
      QVH_HIP(hipMemcpyAsync(nvec.ptr, vectors, count * h->dim * sizeof(float), hipMemcpyHostToDevice, s));
    }
    QVH_HIP(hipGetLastError());
    QVH_HIP(hipStreamSynchronize(s));
    std::swap(h->codes.ptr, ncodes.ptr);
    std::swap(h->codes.bytes, ncodes.bytes);
    std::swap(h->t1.ptr, nt1.ptr);
    std::swap(h->t1.bytes, nt1.bytes);
    std::swap(h->vec.ptr, nvec.ptr);
    std::swap(h->vec.bytes, nvec.bytes);
    std::swap(h->off.ptr, noff.ptr);
    std::swap(h->off.bytes, noff.bytes);
    h->h_off.assign(offsets, offsets + nl + 1);
    h->count = count;
  });
}

uint64_t qvh_ivfpq_size(const qvh_ivfpq* h) { return h ? h->count : 0; }

qvh_status qvh_ivfpq_list_offsets(qvh_ivfpq* h, uint64_t* offsets) {
  return guarded([&] {
    QVH_REQUIRE(h && offsets, "qvh_ivfpq_list_offsets: null argument");
    std::lock_guard<std::mutex> lock(h->mu);
    std::memcpy(offsets, h->h_off.data(), h->h_off.size() * sizeof(uint64_t));
  });
}

qvh_status qvh_ivfpq_lists(qvh_ivfpq* h, uint8_t* codes, float* vectors) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_lists: null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_HIP(hipSetDevice(h->device));
    if (codes && h->count) {
      std::vector<uint8_t> padded(h->count * h->mp);
      QVH_HIP(hipMemcpy(padded.data(), h->codes.ptr, padded.size(), hipMemcpyDeviceToHost));
      for (uint64_t i = 0; i < h->count; ++i) std::memcpy(codes + i * h->m, padded.data() + i * h->mp, h->m);
    }
    if (vectors && h->count) {
      QVH_REQUIRE(h->store_vectors, "vectors are not stored (store_vectors is off)");
      QVH_HIP(hipMemcpy(vectors, h->vec.ptr, h->count * h->dim * sizeof(float), hipMemcpyDeviceToHost));
    }
  });
}

qvh_status qvh_ivfpq_search(qvh_ivfpq* h, const float* queries, uint64_t nq, uint32_t k, uint32_t nprobe,
                            uint64_t refine_factor, const uint64_t* pos_bitmap, uint64_t* out_refs,
                            float* out_dist) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_search: null handle");
    if (nq == 0 || k == 0) return;
    QVH_REQUIRE(queries && out_refs && out_dist, "qvh_ivfpq_search: null buffer");
    std::lock_guard<std::mutex> lock(h->mu);
    if (!h->trained || h->count == 0) {
      for (uint64_t i = 0; i < nq * k; ++i) {
        out_refs[i] = QVH_EMPTY_REF;
        out_dist[i] = __builtin_huge_valf();
      }
      return;
    }
    QVH_HIP(hipSetDevice(h->device));
    hipStream_t s = h->stream;
    float* dq = static_cast<float*>(h->w_q.reserve(nq * h->dim * sizeof(float)));
    QVH_HIP(hipMemcpyAsync(dq, queries, nq * h->dim * sizeof(float), hipMemcpyHostToDevice, s));
    const uint64_t* dbits = nullptr;
    if (pos_bitmap) {
      const size_t words = ceil_div(h->count, 64);
      uint64_t* b = static_cast<uint64_t*>(h->w_bits.reserve(words * sizeof(uint64_t)));
      QVH_HIP(hipMemcpyAsync(b, pos_bitmap, words * sizeof(uint64_t), hipMemcpyHostToDevice, s));
      dbits = b;
    }
    uint64_t* drefs = static_cast<uint64_t*>(h->w_refs.reserve(nq * k * sizeof(uint64_t)));
    float* ddist = static_cast<float*>(h->w_dist.reserve(nq * k * sizeof(float)));
    h->timed = h->timing > 0;
    h->timed_bytes = h->timing > 1;
    ivf_search_impl(h, dq, nq, k, nprobe, refine_factor, dbits, drefs, ddist, s);
    QVH_HIP(hipMemcpyAsync(out_refs, drefs, nq * k * sizeof(uint64_t), hipMemcpyDeviceToHost, s));
    QVH_HIP(hipMemcpyAsync(out_dist, ddist, nq * k * sizeof(float), hipMemcpyDeviceToHost, s));
    QVH_HIP(hipStreamSynchronize(s));
  });
}

qvh_status qvh_ivfpq_search_device(qvh_ivfpq* h, const float* d_queries, uint64_t nq, uint32_t k,
                                   uint32_t nprobe, uint64_t refine_factor, const uint64_t* d_pos_bitmap,
                                   uint64_t* d_out_refs, float* d_out_dist, void* stream) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_search_device: null handle");
    if (nq == 0 || k == 0) return;
    QVH_REQUIRE(d_queries && d_out_refs && d_out_dist, "qvh_ivfpq_search_device: null buffer");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_REQUIRE(h->trained && h->count > 0, "qvh_ivfpq_search_device: index is untrained or empty");
    QVH_HIP(hipSetDevice(h->device));
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : h->stream;
    h->timed = h->timing > 0;
    h->timed_bytes = h->timing > 1;
    on_handle_timeline(h->stream, h->join, s, [&](hipStream_t st) {
      ivf_search_impl(h, d_queries, nq, k, nprobe, refine_factor, d_pos_bitmap, d_out_refs, d_out_dist, st);
    });
  });
}

qvh_status qvh_ivfpq_set_timing(qvh_ivfpq* h, int enable) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_set_timing: null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_HIP(hipSetDevice(h->device));
    QVH_REQUIRE(enable >= 0 && enable <= 2, "qvh_ivfpq_set_timing: level must be 0, 1 or 2");
    if (enable && !h->ev[0]) {
      for (hipEvent_t& e : h->ev) QVH_HIP(hipEventCreate(&e));
    }
    h->timing = enable;
  });
}

qvh_status qvh_ivfpq_last_timing(qvh_ivfpq* h, float* select_ms, float* scan_ms, uint64_t* code_bytes) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_last_timing: null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_REQUIRE(h->timed, "qvh_ivfpq_last_timing: the last search was not timed");
    QVH_HIP(hipSetDevice(h->device));
    QVH_HIP(hipEventSynchronize(h->ev[2]));
    float a = 0, b = 0;
    QVH_HIP(hipEventElapsedTime(&a, h->ev[0], h->ev[1]));
    QVH_HIP(hipEventElapsedTime(&b, h->ev[1], h->ev[2]));
    if (select_ms) *select_ms = a;
    if (scan_ms) *scan_ms = b;
    if (code_bytes) {
      QVH_REQUIRE(h->timed_bytes, "qvh_ivfpq_last_timing: code bytes are measured at timing level 2");
      QVH_HIP(hipStreamSynchronize(h->stream));
      QVH_HIP(hipMemcpy(code_bytes, h->w_bytes.ptr, sizeof(uint64_t), hipMemcpyDeviceToHost));
    }
  });
}

qvh_status qvh_ivfpq_last_fallbacks(qvh_ivfpq* h, uint32_t* count) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr && count != nullptr, "qvh_ivfpq_last_fallbacks: null argument");
    std::lock_guard<std::mutex> lock(h->mu);
    QVH_HIP(hipSetDevice(h->device));
    *count = 0;
    if (!h->last_certified) return;
    QVH_HIP(hipStreamSynchronize(h->stream));
    QVH_HIP(hipMemcpy(count, h->w_fb.ptr, sizeof(uint32_t), hipMemcpyDeviceToHost));
  });
}

qvh_status qvh_ivfpq_sync(qvh_ivfpq* h) {
  return guarded([&] {
    QVH_REQUIRE(h != nullptr, "qvh_ivfpq_sync: null handle");
    QVH_HIP(hipSetDevice(h->device));
    QVH_HIP(hipStreamSynchronize(h->stream));
  });
}

// ---- point sets for k-means assignment ------------------------------------------------------------

struct qvh_points {
  uint64_t n = 0;
  uint32_t dim = 0;
  int device = 0;
  DeviceBuffer x, cent, ct, norms, out, fb;
  AssignTable asg;
  std::mutex mu;
};

qvh_status qvh_points_create(const float* x, uint64_t n, uint32_t dim, qvh_points** out) {
  return guarded([&] {
    QVH_REQUIRE(out != nullptr, "qvh_points_create: null output");
    *out = nullptr;
    QVH_REQUIRE(dim >= 1, "qvh_points_create: dim must be positive");
    QVH_REQUIRE(x != nullptr || n == 0, "qvh_points_create: null points");
    const int dev = current_device();
    auto* p = new qvh_points;
    p->n = n;
    p->dim = dim;
    p->device = dev;
    try {
      p->x.reserve(std::max<uint64_t>(n, 1) * dim * sizeof(float));
      if (n) QVH_HIP(hipMemcpy(p->x.ptr, x, n * dim * sizeof(float), hipMemcpyHostToDevice));
    } catch (...) {
      delete p;
      throw;
    }
    *out = p;
  });
}

void qvh_points_destroy(qvh_points* p) { delete p; }

qvh_status qvh_points_nearest(qvh_points* p, const float* centroids, uint32_t k, int max_inner_product,
                              uint32_t* out_assign) {
  return guarded([&] {
    QVH_REQUIRE(p && centroids && out_assign, "qvh_points_nearest: null argument");
    QVH_REQUIRE(k >= 1, "qvh_points_nearest: k must be positive");
    std::lock_guard<std::mutex> lock(p->mu);
    QVH_HIP(hipSetDevice(p->device));
    if (p->n == 0) return;
    const uint64_t cb = static_cast<uint64_t>(k) * p->dim * sizeof(float);
    p->cent.reserve(cb);
    p->ct.reserve(cb);
    p->norms.reserve(k * sizeof(float));
    p->out.reserve(p->n * sizeof(uint32_t));
    QVH_HIP(hipMemcpy(p->cent.ptr, centroids, cb, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(centroid_prep_kernel, dim3(static_cast<unsigned>(ceil_div(k, 256))), dim3(256), 0, nullptr,
                       p->cent.as<float>(), k, p->dim, p->ct.as<float>(), p->norms.as<float>());
    NearestArgs na{};
    na.x = p->x.as<float>();
    na.n = p->n;
    na.dim = p->dim;
    na.x_stride = p->dim;
    na.ct = p->ct.as<float>();
    na.norms = p->norms.as<float>();
    na.k = k;
    na.max_ip = max_inner_product;
    na.out32 = p->out.as<uint32_t>();
    prepare_assign_table(p->asg, p->cent.as<float>(), p->norms.as<float>(), k, p->dim, max_inner_product, nullptr);
    launch_assign(na, p->asg, p->fb, nullptr);
    QVH_HIP(hipMemcpy(out_assign, p->out.ptr, p->n * sizeof(uint32_t), hipMemcpyDeviceToHost));
  });
}

}  // extern "C"
