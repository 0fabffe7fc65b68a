// Wave-level top-k selection over 64-bit keys (ordered float distance << 32 | id), shared by the
// scans that cannot keep their candidates in registers.
//
// A wave appends candidates to a private LDS queue of CAP keys. A cut keeps the `keep` smallest
// keys: the keep-th smallest distance t is found bit by bit with wave ballots (32 steps), every
// key with distance < t is kept, and among the keys at distance t only the smallest ids that make
// up exactly `keep` (a second 32-step search on the id bits, needed only when ties would otherwise
// keep more than CAP / 2). The wave's keep-th distance bounds the final keep-th distance from
// above, so candidates beyond it can be dropped as they arrive.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace qvh {

/// Ascending bitonic sort of N * 64 keys held by one wave, element e = i * 64 + lane in k[i].
template <int N>
__device__ __forceinline__ void wave_sort(uint64_t (&k)[N]) {
  const int lane = threadIdx.x & 63;
  constexpr int total = N * 64;
#pragma unroll
  for (int size = 2; size <= total; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= 64) {
        const int is = stride / 64;
#pragma unroll
        for (int i = 0; i < N; ++i) {
          const int j = i ^ is;
          if (j > i) {
            const bool up = ((i * 64) & size) == 0;
            const uint64_t x = k[i], y = k[j];
            const bool swap = (x > y) == up;
            k[i] = swap ? y : x;
            k[j] = swap ? x : y;
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < N; ++i) {
          const uint64_t other = lane_xor_u64(k[i], stride);
          const bool up = ((i * 64 + lane) & size) == 0;
          const bool lower = (lane & stride) == 0;
          k[i] = (lower == up) ? (other < k[i] ? other : k[i]) : (other > k[i] ? other : k[i]);
        }
      }
    }
  }
}

/// Ascending bitonic sort of N * 64 32-bit values held by one wave, element e = i * 64 + lane in
/// k[i] (duplicates allowed).
template <int N>
__device__ __forceinline__ void wave_sort_u32(uint32_t (&k)[N]) {
  const int lane = threadIdx.x & 63;
  constexpr int total = N * 64;
#pragma unroll
  for (int size = 2; size <= total; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= 64) {
        const int is = stride / 64;
#pragma unroll
        for (int i = 0; i < N; ++i) {
          const int j = i ^ is;
          if (j > i) {
            const bool up = ((i * 64) & size) == 0;
            const uint32_t x = k[i], y = k[j];
            k[i] = up ? min(x, y) : max(x, y);
            k[j] = up ? max(x, y) : min(x, y);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < N; ++i) {
          const uint32_t other = lane_xor_u32(k[i], stride);
          const bool up = ((i * 64 + lane) & size) == 0;
          const bool lower = (lane & stride) == 0;
          k[i] = (lower == up) ? min(other, k[i]) : max(other, k[i]);
        }
      }
    }
  }
}

/// Ascending sort of a bitonic sequence of N * 64 keys held by one wave (element e = i * 64 + lane
/// in k[i]): the last merge stage of the bitonic sort.
template <int N>
__device__ __forceinline__ void wave_merge(uint64_t (&k)[N]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int stride = N * 32; stride > 0; stride >>= 1) {
    if (stride >= 64) {
      const int is = stride / 64;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ is;
        if (j > i) {
          const uint64_t x = k[i], y = k[j];
          k[i] = x < y ? x : y;
          k[j] = x < y ? y : x;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const uint64_t other = lane_xor_u64(k[i], stride);
        const bool lower = (lane & stride) == 0;
        k[i] = lower ? (other < k[i] ? other : k[i]) : (other > k[i] ? other : k[i]);
      }
    }
  }
}

/// Key at sorted position e (wave-uniform) of a wave-sorted register array.
template <int N>
__device__ __forceinline__ uint64_t wave_key_at(const uint64_t (&k)[N], uint32_t e) {
  uint64_t v = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (static_cast<uint32_t>(i) == e / 64) v = k[i];
  }
  return __shfl(v, static_cast<int>(e % 64), 64);
}


__device__ __forceinline__ uint32_t lane_rank(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

/// Cuts queue[0, cnt) (wave-uniform cnt) to its `keep` smallest keys; returns the new count and
/// the keep-th smallest distance (ordered bits) in *bound, or leaves both alone when cnt <= keep.
template <int CAP>
__device__ uint32_t wave_cut(uint64_t* queue, uint32_t cnt, uint32_t keep, uint32_t* bound) {
  constexpr int QN = CAP / 64;
  const int lane = threadIdx.x & 63;
  if (cnt <= keep) return cnt;
  uint64_t k[QN];
  uint32_t d[QN];
#pragma unroll
  for (int i = 0; i < QN; ++i) {
    const uint32_t e = i * 64 + lane;
    k[i] = e < cnt ? queue[e] : ~0ull;
    d[i] = static_cast<uint32_t>(k[i] >> 32);
  }
  uint32_t t = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t probe = t | ((1u << b) - 1u);
    uint32_t below = 0;
#pragma unroll
    for (int i = 0; i < QN; ++i) {
      if (static_cast<uint32_t>(i * 64) < cnt) below += static_cast<uint32_t>(__popcll(__ballot(d[i] <= probe)));
    }
    if (below < keep) t |= 1u << b;
  }
  uint32_t kept = 0, under = 0;
#pragma unroll
  for (int i = 0; i < QN; ++i) {
    if (static_cast<uint32_t>(i * 64) < cnt) {
      kept += static_cast<uint32_t>(__popcll(__ballot(d[i] <= t)));
      under += static_cast<uint32_t>(__popcll(__ballot(d[i] < t)));
    }
  }
  uint32_t u = 0xFFFFFFFFu;
  if (kept > static_cast<uint32_t>(CAP / 2)) {
    const uint32_t need = keep - under;
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
      if (keepit) queue[at + lane_rank(mk)] = k[i];
      at += static_cast<uint32_t>(__popcll(mk));
    }
  }
  __builtin_amdgcn_wave_barrier();
  *bound = t;
  return at;
}

/// Ascending bitonic sort of s[0, n) (n a power of two) by the whole block.
__device__ __forceinline__ void block_sort_keys(uint64_t* s, uint32_t n) {
  for (uint32_t size = 2; size <= n; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (uint32_t i = threadIdx.x; i < n / 2; i += blockDim.x) {
        const uint32_t lo = 2 * i - (i & (stride - 1));
        const uint32_t hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t x = s[lo], y = s[hi];
        if ((x > y) == up) {
          s[lo] = y;
          s[hi] = x;
        }
      }
    }
  }
  __syncthreads();
}

}  // namespace qvh
