// LDS tile staging for the fused kernels.
//
// A tile is ROWS time steps x COLS columns (channels or states) of a (B, L, C) strided
// tensor.  Thread e of the workgroup handles tile elements e, e + 256, ...; the element ->
// (row, col) map puts consecutive threads on consecutive addresses of whichever axis has
// unit stride (`cfast` = column axis contiguous, else time axis), so the global reads and
// writes of every layout the reference produces -- time-major (B,L,D) and the channel-major
// (B,D,L) views of models/mamba.py:101,107 -- are coalesced.  Out-of-range rows/columns
// load as 0, which is an identity step of the recurrence (delta = 0 gives a = 1, b = 0).
#pragma once

#include "ssm_device.hpp"
#include "ssm_internal.hpp"

namespace ssm {

template <typename CT> struct TileCfg;
template <> struct TileCfg<float> {
  static constexpr int CK = 32;  // time steps per chunk (= checkpoint interval)
  static constexpr int RS = 8;   // steps per LDS reduction round
};
template <> struct TileCfg<double> {
  static constexpr int CK = 16;
  static constexpr int RS = 2;
};

template <typename T>
__device__ __forceinline__ const T *vp(const KView &v) { return (const T *)v.p; }
template <typename T>
__device__ __forceinline__ T *vpw(const KView &v) { return (T *)v.p; }
template <typename CT>
__device__ __forceinline__ CT vload(const KView &v, int64_t off) { return ((const CT *)v.p)[off]; }
template <typename CT>
__device__ __forceinline__ void vstore(const KView &v, int64_t off, CT val) { ((CT *)v.p)[off] = val; }

template <int ROWS, int COLS>
__device__ __forceinline__ void tile_rc(int idx, bool cfast, int &r, int &c) {
  if (cfast) {
    r = idx / COLS;
    c = idx % COLS;
  } else {
    r = idx % ROWS;
    c = idx / ROWS;
  }
}

template <typename IT, typename CT, int ROWS, int COLS>
struct TileLoad {
  static constexpr int E = (ROWS * COLS + kThreads - 1) / kThreads;
  CT v[E];

  __device__ __forceinline__ void load(const KView &V, int64_t b, int t0, int L, int c0, int C,
                                       bool cfast) {
    const IT *base = vp<IT>(V) + b * V.s0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int idx = threadIdx.x + e * kThreads;
      int r, c;
      tile_rc<ROWS, COLS>(idx, cfast, r, c);
      const int t = t0 + r, cc = c0 + c;
      CT val = 0;
      if (idx < ROWS * COLS && t < L && cc < C)
        val = Conv<IT>::load(base + (int64_t)t * V.s1 + (int64_t)cc * V.s2);
      v[e] = val;
    }
  }

  __device__ __forceinline__ void store(CT (*S)[COLS], bool cfast) const {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int idx = threadIdx.x + e * kThreads;
      if (idx >= ROWS * COLS) break;
      int r, c;
      tile_rc<ROWS, COLS>(idx, cfast, r, c);
      S[r][c] = v[e];
    }
  }
};

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

// Store a staged tile transposed: element (row r = time, col c) -> S[c][r] (rows padded to RP).
template <typename IT, typename CT, int ROWS, int COLS, int RP>
__device__ __forceinline__ void store_t(const TileLoad<IT, CT, ROWS, COLS> &tl, CT (*S)[RP], bool cfast) {
#pragma unroll
  for (int e = 0; e < TileLoad<IT, CT, ROWS, COLS>::E; ++e) {
    const int idx = threadIdx.x + e * kThreads;
    if (idx >= ROWS * COLS) break;
    int r, c;
    tile_rc<ROWS, COLS>(idx, cfast, r, c);
    S[c][r] = tl.v[e];
  }
}

// delta' = softplus(delta + bias) (parts optional) for in-range elements; padding stays 0.
// Stored transposed (S[col][time]); when `sg` is given it receives sigmoid(delta + bias), the
// derivative of the softplus (1 without softplus).
template <typename IT, typename CT, int ROWS, int COLS, int RP>
__device__ __forceinline__ void store_delta(const TileLoad<IT, CT, ROWS, COLS> &tl, CT (*S)[RP],
                                            CT (*sg)[RP], bool cfast, int has_bias, int softplus,
                                            const KView &bias, int c0, int C, int t0, int L) {
#pragma unroll
  for (int e = 0; e < TileLoad<IT, CT, ROWS, COLS>::E; ++e) {
    const int idx = threadIdx.x + e * kThreads;
    if (idx >= ROWS * COLS) break;
    int r, c;
    tile_rc<ROWS, COLS>(idx, cfast, r, c);
    CT v = tl.v[e], g = 1;
    if (t0 + r < L && c0 + c < C) {
      if (has_bias) v += vload<CT>(bias, (int64_t)(c0 + c) * bias.s0);
      if (softplus) {
        g = sigmoid_ct<CT>(v);
        v = softplus_ct<CT>(v);
      }
    }
    S[c][r] = v;
    if (sg) sg[c][r] = g;
  }
}

}  // namespace ssm
