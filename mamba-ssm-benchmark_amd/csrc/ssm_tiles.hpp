// Typed access to strided views (KView) and vector reads of LDS rows, shared by the kernels.
#pragma once

#include "ssm_device.hpp"
#include "ssm_internal.hpp"

namespace ssm {

template <typename T>
__device__ __forceinline__ const T *vp(const KView &v) { return (const T *)v.p; }
template <typename T>
__device__ __forceinline__ T *vpw(const KView &v) { return (T *)v.p; }
template <typename CT>
__device__ __forceinline__ CT vload(const KView &v, int64_t off) { return ((const CT *)v.p)[off]; }
template <typename CT>
__device__ __forceinline__ void vstore(const KView &v, int64_t off, CT val) { ((CT *)v.p)[off] = val; }

// Vector load of N consecutive CT values from a 16-byte aligned LDS address.
template <typename CT, int N>
__device__ __forceinline__ void lds_row(const CT *src, CT (&dst)[N]) {
  constexpr int V = 16 / sizeof(CT);
  typedef CT vec __attribute__((ext_vector_type(V)));
  static_assert(N % V == 0, "row length must be a multiple of the vector width");
#pragma unroll
  for (int j = 0; j < N / V; ++j) {
    const vec v = *reinterpret_cast<const vec *>(src + j * V);
#pragma unroll
    for (int k = 0; k < V; ++k) dst[j * V + k] = v[k];
  }
}

// Sum of N values in pairwise order (N a power of two): the same adds as a running sum, with
// rounding that grows with log2(N) rather than N and independent adds for the scheduler.
template <int N>
__device__ __forceinline__ float pairwise_sum(const float (&v)[N]) {
  static_assert((N & (N - 1)) == 0, "power of two");
  if constexpr (N == 1) {
    return v[0];
  } else {
    float h[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) h[i] = v[2 * i] + v[2 * i + 1];
    return pairwise_sum<N / 2>(h);
  }
}

// Dot product of two N-vectors (N a multiple of 4) as four interleaved FMA chains over
// j = i mod 4, added pairwise at the end: one instruction per term, four independent chains.
template <int N>
__device__ __forceinline__ float dot_sum(const float (&a)[N], const float (&w)[N]) {
  static_assert(N % 4 == 0 && N >= 4, "dot_sum length");
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = a[i] * w[i];
#pragma unroll
  for (int j = 4; j < N; j += 4)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = fmaf(a[j + i], w[j + i], s[i]);
  return (s[0] + s[1]) + (s[2] + s[3]);
}

// Sum of count values at src[0], src[stride], ... in index order (the bits of a running sum),
// the reads of G terms issued together ahead of their adds: a sum over partials in HBM is
// otherwise a chain of dependent memory round trips.
// ST: the running sum's type (a float64 sum of float32 partials keeps a long sum's rounding from
// growing with the count).
template <int G, typename CT, typename ST = CT>
__device__ inline ST ordered_sum(const CT *src, int64_t stride, int64_t count) {
  ST s = 0;
  int64_t k = 0;
  for (; k + G <= count; k += G) {
    CT v[G];
#pragma unroll
    for (int u = 0; u < G; ++u) v[u] = src[(k + u) * stride];
#pragma unroll
    for (int u = 0; u < G; ++u) s += (ST)v[u];
  }
  for (; k < count; ++k) s += (ST)src[k * stride];
  return s;
}

}  // namespace ssm
