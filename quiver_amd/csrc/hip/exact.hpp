// Device restatements of the reference's x86-64 float arithmetic, bit for bit.
//
// The reference's flat scan, refine and normalize use its AVX2+FMA kernels
// (src/simd/kernels_avx2.cc:35-83, chosen by src/simd/dispatch.cc:108-117 on any x86-64 CPU with
// AVX2 and FMA). Their reduction order is: four 8-lane FMA accumulators over blocks of 32
// elements, an 8-wide loop into the first accumulator, the horizontal sum
// ((s0+s1)+(s2+s3)) -> lo[j] = v[j]+v[j+4] -> (lo0+lo1)+(lo2+lo3), then a scalar tail of fewer
// than 8 elements which GCC 11 -O3 compiles as: the first four products separately rounded and
// added in order, the remaining ones fused. One GPU thread replays that sequence exactly.
//
// All qvh sources are compiled with -ffp-contract=off, so every a*b+c written here is two
// roundings; fused steps are explicit fmaf().
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qvh {

__device__ __forceinline__ float avx2_reduce(const float (&s)[4][8]) {
  float v[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) v[l] = (s[0][l] + s[1][l]) + (s[2][l] + s[3][l]);
  float lo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) lo[j] = v[j] + v[j + 4];
  return (lo[0] + lo[1]) + (lo[2] + lo[3]);
}

/// sum_i (a_i - b_i)^2 in the order of src/simd/kernels_avx2.cc:35-56.
__device__ inline float exact_l2sqr(const float* __restrict__ a, const float* __restrict__ b,
                                    uint32_t dim) {
  float s[4][8];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int l = 0; l < 8; ++l) s[u][l] = 0.0f;
  uint32_t i = 0;
  for (; i + 32 <= dim; i += 32) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const float d = a[i + 8 * u + l] - b[i + 8 * u + l];
        s[u][l] = fmaf(d, d, s[u][l]);
      }
  }
  for (; i + 8 <= dim; i += 8) {
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const float d = a[i + l] - b[i + l];
      s[0][l] = fmaf(d, d, s[0][l]);
    }
  }
  float sum = avx2_reduce(s);
  const uint32_t v4 = i + (dim - i) / 4 * 4;
  for (; i < v4; ++i) {
    const float d = a[i] - b[i];
    sum = sum + d * d;
  }
  for (; i < dim; ++i) {
    const float d = a[i] - b[i];
    sum = fmaf(d, d, sum);
  }
  return sum;
}

/// sum_i a_i * b_i in the order of src/simd/kernels_avx2.cc:58-83.
__device__ inline float exact_dot(const float* __restrict__ a, const float* __restrict__ b,
                                  uint32_t dim) {
  float s[4][8];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int l = 0; l < 8; ++l) s[u][l] = 0.0f;
  uint32_t i = 0;
  for (; i + 32 <= dim; i += 32) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int l = 0; l < 8; ++l) s[u][l] = fmaf(a[i + 8 * u + l], b[i + 8 * u + l], s[u][l]);
  }
  for (; i + 8 <= dim; i += 8) {
#pragma unroll
    for (int l = 0; l < 8; ++l) s[0][l] = fmaf(a[i + l], b[i + l], s[0][l]);
  }
  float sum = avx2_reduce(s);
  const uint32_t v4 = i + (dim - i) / 4 * 4;
  for (; i < v4; ++i) sum = sum + a[i] * b[i];
  for (; i < dim; ++i) sum = fmaf(a[i], b[i], sum);
  return sum;
}

/// exact_l2sqr (L2) or exact_dot of one pair by an aligned group of eight lanes, bit for bit: lane l
/// of the group holds lane l of the four 8-lane accumulators, the horizontal sum takes the same
/// association through lane exchanges inside the group, and lane 0 of the group adds the scalar
/// tail and returns the sum (the other lanes' results are meaningless). Every lane of the wave must
/// call it together; lanes with valid == false read nothing.
template <bool L2>
__device__ inline float exact_group8(const float* __restrict__ a, const float* __restrict__ b, uint32_t dim,
                                     bool valid) {
  const uint32_t l = threadIdx.x & 7u;
  auto term = [](float x, float y, float s) {
    if constexpr (L2) {
      const float d = x - y;
      return fmaf(d, d, s);
    } else {
      return fmaf(x, y, s);
    }
  };
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  const uint32_t n8 = dim / 8 * 8;  // where the 32- and 8-element loops of exact_l2sqr stop
  if (valid) {
    uint32_t i = 0;
    for (; i + 32 <= dim; i += 32) {
      s0 = term(a[i + l], b[i + l], s0);
      s1 = term(a[i + 8 + l], b[i + 8 + l], s1);
      s2 = term(a[i + 16 + l], b[i + 16 + l], s2);
      s3 = term(a[i + 24 + l], b[i + 24 + l], s3);
    }
    for (; i < n8; i += 8) s0 = term(a[i + l], b[i + l], s0);
  }
  const float v = (s0 + s1) + (s2 + s3);      // v[l]
  const float lo = v + __shfl_down(v, 4, 8);  // lo[j] = v[j] + v[j + 4] on lanes 0..3
  const float t = lo + __shfl_xor(lo, 1, 8);  // lo0 + lo1 on lane 0, lo2 + lo3 on lane 2
  float sum = t + __shfl_xor(t, 2, 8);        // (lo0 + lo1) + (lo2 + lo3) on lane 0
  if (valid && l == 0) {
    uint32_t i = n8;
    const uint32_t v4 = i + (dim - i) / 4 * 4;
    for (; i < v4; ++i) {
      if constexpr (L2) {
        const float d = a[i] - b[i];
        sum = sum + d * d;
      } else {
        sum = sum + a[i] * b[i];
      }
    }
    for (; i < dim; ++i) sum = term(a[i], b[i], sum);
  }
  return sum;
}

/// exact_group8 for NC pairs (a, b[c]) at once, with the same arithmetic for each: the elements of
/// a are loaded once for all NC, and the NC rows' loads go out together. Every b[c] must point at
/// dim readable floats (a slot without a row may pass a itself and ignore its result). Lane 0 of
/// the group returns the NC sums in out.
template <bool L2, int NC>
__device__ inline void exact_group8_n(const float* __restrict__ a, const float* const (&b)[NC], uint32_t dim,
                                      float (&out)[NC]) {
  const uint32_t l = threadIdx.x & 7u;
  auto term = [](float x, float y, float s) {
    if constexpr (L2) {
      const float d = x - y;
      return fmaf(d, d, s);
    } else {
      return fmaf(x, y, s);
    }
  };
  float s[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u) s[c][u] = 0.0f;
  const uint32_t n8 = dim / 8 * 8;  // where the 32- and 8-element loops of exact_l2sqr stop
  uint32_t i = 0;
  for (; i + 32 <= dim; i += 32) {
    float av[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) av[u] = a[i + 8 * u + l];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u) s[c][u] = term(av[u], b[c][i + 8 * u + l], s[c][u]);
  }
  for (; i < n8; i += 8) {
    const float a0 = a[i + l];
#pragma unroll
    for (int c = 0; c < NC; ++c) s[c][0] = term(a0, b[c][i + l], s[c][0]);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float v = (s[c][0] + s[c][1]) + (s[c][2] + s[c][3]);  // v[l]
    const float lo = v + __shfl_down(v, 4, 8);                   // lo[j] = v[j] + v[j + 4] on lanes 0..3
    const float t = lo + __shfl_xor(lo, 1, 8);                   // lo0 + lo1 on lane 0, lo2 + lo3 on lane 2
    float sum = t + __shfl_xor(t, 2, 8);                         // (lo0 + lo1) + (lo2 + lo3) on lane 0
    if (l == 0) {
      uint32_t k = n8;
      const uint32_t v4 = k + (dim - k) / 4 * 4;
      for (; k < v4; ++k) {
        if constexpr (L2) {
          const float d = a[k] - b[c][k];
          sum = sum + d * d;
        } else {
          sum = sum + a[k] * b[c][k];
        }
      }
      for (; k < dim; ++k) sum = term(a[k], b[c][k], sum);
    }
    out[c] = sum;
  }
}

/// simd::normalize (src/simd/dispatch.cc:119-135) of one row in place.
__device__ inline void exact_normalize(float* v, uint32_t dim) {
  const float norm_sq = exact_dot(v, v, dim);
  if (!isfinite(norm_sq)) {
    double acc = 0.0;
    for (uint32_t i = 0; i < dim; ++i) acc = acc + static_cast<double>(v[i]) * static_cast<double>(v[i]);
    const double inv = acc > 0.0 && isfinite(acc) ? 1.0 / sqrt(acc) : 0.0;
    if (inv == 0.0) return;
    for (uint32_t i = 0; i < dim; ++i) v[i] = static_cast<float>(static_cast<double>(v[i]) * inv);
    return;
  }
  if (norm_sq <= 0.0f) return;
  const float inv = 1.0f / sqrtf(norm_sq);
  for (uint32_t i = 0; i < dim; ++i) v[i] = v[i] * inv;
}

/// The flat scan's distance (src/flat_index.cc:87-88): squared L2, or 1 - dot for inner product
/// and cosine; NaN becomes +inf.
__device__ inline float exact_flat_distance(const float* q, const float* x, uint32_t dim, bool l2) {
  const float d = l2 ? exact_l2sqr(q, x, dim) : 1.0f - exact_dot(q, x, dim);
  return d == d ? d : __builtin_huge_valf();
}

}  // namespace qvh
