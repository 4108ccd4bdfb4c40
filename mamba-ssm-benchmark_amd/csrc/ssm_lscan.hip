// Linear-recurrence scan algorithms for gfx950: h_t = a_t h_{t-1} + b_t over (B, L, M).
//
// Replaces the four torch scans of models/scan.py with kernels that keep each algorithm's
// structure (so `scan=` still selects an algorithm, as in the reference's SCANS registry,
// models/scan.py:168-173):
//   sequential     models/scan.py:70-76    one lane per (b, m) walks the sequence.
//   hillis_steele  models/scan.py:87-98    a 256-lane workgroup per (b, m) runs recursive
//                                          doubling over tiles of 256 steps in LDS; the state
//                                          entering a tile is folded into its first element
//                                          (as _fold_h0 does with h0, :79-84).
//   blelloch       models/scan.py:101-135  up-sweep / down-sweep over tiles of 512 steps in
//                                          LDS, giving exclusive (A, S) prefixes; h = a (A h_in
//                                          + S) + b, the tile's last h carried to the next.
//   chunked        models/scan.py:142-165  three launches: per-chunk local scans from zero
//                                          (chunk summaries P = prod a, E = local end), a scan
//                                          over the chunk summaries per (b, m), then the
//                                          correction h += (prod of a inside the chunk) h_in.
// Direction: with `reverse` the recurrence runs from t = L-1 down to 0.  With `shift` (used
// by the adjoint) the multiplier at a step is the a of the previous step in processing order
// and 1 for the first step: lambda_t = g_t + a_{t+1} lambda_{t+1} (models/scan.py:239-240).
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"

namespace ssm {

template <typename CT>
struct Chain {
  const LscanParams &P;
  int64_t b, m;
  __device__ __forceinline__ int t_of(int pos) const { return P.reverse ? (int)P.L - 1 - pos : pos; }
  __device__ __forceinline__ CT a_at(int t) const {
    return vload<CT>(P.a, b * P.a.s0 + (int64_t)t * P.a.s1 + m * P.a.s2);
  }
  // multiplier used at processing position pos
  __device__ __forceinline__ CT mult(int pos) const {
    if (!P.shift) return a_at(t_of(pos));
    return pos > 0 ? a_at(t_of(pos - 1)) : (CT)1;
  }
  __device__ __forceinline__ CT b_at(int t) const {
    return vload<CT>(P.b, b * P.b.s0 + (int64_t)t * P.b.s1 + m * P.b.s2);
  }
  __device__ __forceinline__ int64_t h_off(int t) const { return b * P.h.s0 + (int64_t)t * P.h.s1 + m * P.h.s2; }
  __device__ __forceinline__ CT h0() const {
    return P.h0.p ? vload<CT>(P.h0, b * P.h0.s0 + m * P.h0.s1) : (CT)0;
  }
};

// ------------------------------------------------------------------ sequential
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_seq(const LscanParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.M) return;
  Chain<CT> ch{P, i / P.M, i % P.M};
  CT h = ch.h0();
  for (int pos = 0; pos < (int)P.L; ++pos) {
    const int t = ch.t_of(pos);
    h = fma(ch.mult(pos), h, ch.b_at(t));
    vstore<CT>(P.h, ch.h_off(t), h);
  }
}

// ------------------------------------------------------------------ Hillis-Steele
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_hs(const LscanParams P) {
  constexpr int T = 256;
  __shared__ CT sA[2][T], sS[2][T];
  Chain<CT> ch{P, (int64_t)blockIdx.y, (int64_t)blockIdx.x};
  const int j = threadIdx.x;
  CT carry = ch.h0();
  for (int base = 0; base < (int)P.L; base += T) {
    const int pos = base + j;
    const bool valid = pos < (int)P.L;
    CT A = valid ? ch.mult(pos) : (CT)1;
    CT S = valid ? ch.b_at(ch.t_of(pos)) : (CT)0;
    if (j == 0) S = fma(A, carry, S);  // fold the incoming state into the first element
    int cur = 0;
    sA[cur][j] = A;
    sS[cur][j] = S;
    __syncthreads();
    for (int off = 1; off < T; off *= 2) {  // after this step: composition of 2*off elements
      if (j >= off) {
        S = fma(A, sS[cur][j - off], S);
        A = A * sA[cur][j - off];
      }
      sA[cur ^ 1][j] = A;
      sS[cur ^ 1][j] = S;
      cur ^= 1;
      __syncthreads();
    }
    if (valid) vstore<CT>(P.h, ch.h_off(ch.t_of(pos)), S);
    carry = sS[cur][T - 1];
    __syncthreads();
  }
}

// ------------------------------------------------------------------ Blelloch
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_bl(const LscanParams P) {
  constexpr int T = 512;  // elements per tile, two per lane
  __shared__ CT sA[T], sS[T];
  Chain<CT> ch{P, (int64_t)blockIdx.y, (int64_t)blockIdx.x};
  const int j = threadIdx.x;
  CT carry = ch.h0();
  for (int base = 0; base < (int)P.L; base += T) {
    CT a_own[2], b_own[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int k = 2 * j + q, pos = base + k;
      const bool valid = pos < (int)P.L;
      a_own[q] = valid ? ch.mult(pos) : (CT)1;  // padding with the identity (1, 0)
      b_own[q] = valid ? ch.b_at(ch.t_of(pos)) : (CT)0;
      sA[k] = a_own[q];
      sS[k] = b_own[q];
    }
    __syncthreads();
    // up-sweep: right <- right o left
    for (int s = 2; s <= T; s *= 2) {
      const int k = (j + 1) * s - 1;
      if (k < T) {
        const int l = k - s / 2;
        sS[k] = fma(sA[k], sS[l], sS[k]);
        sA[k] = sA[k] * sA[l];
      }
      __syncthreads();
    }
    if (j == 0) {
      sA[T - 1] = 1;
      sS[T - 1] = 0;
    }
    __syncthreads();
    // down-sweep: left <- right; right <- left_old o right
    for (int s = T; s >= 2; s /= 2) {
      const int k = (j + 1) * s - 1;
      if (k < T) {
        const int l = k - s / 2;
        const CT tA = sA[l], tS = sS[l];
        sA[l] = sA[k];
        sS[l] = sS[k];
        sS[k] = fma(sS[k], tA, tS);
        sA[k] = sA[k] * tA;
      }
      __syncthreads();
    }
    // exclusive prefixes: the state entering element k is A_k h_in + S_k
    CT last = 0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int k = 2 * j + q, pos = base + k;
      const CT prev = fma(sA[k], carry, sS[k]);
      const CT h = fma(a_own[q], prev, b_own[q]);
      if (pos < (int)P.L) vstore<CT>(P.h, ch.h_off(ch.t_of(pos)), h);
      if (k == T - 1) last = h;
    }
    __syncthreads();
    if (j == blockDim.x - 1) sS[0] = last;  // broadcast the tile's last state
    __syncthreads();
    carry = sS[0];
    __syncthreads();
  }
}

// ------------------------------------------------------------------ chunked (three phases)
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_chunk_local(const LscanParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.nc * P.M) return;
  const int64_t m = i % P.M, cj = (i / P.M) % P.nc, b = i / (P.M * P.nc);
  Chain<CT> ch{P, b, m};
  CT h = 0, prod = 1;
  const int p0 = (int)cj * P.chunk;
  for (int pos = p0; pos < p0 + P.chunk && pos < (int)P.L; ++pos) {
    const CT a = ch.mult(pos);
    h = fma(a, h, ch.b_at(ch.t_of(pos)));
    prod *= a;
    vstore<CT>(P.h, ch.h_off(ch.t_of(pos)), h);
  }
  CT *ws = (CT *)P.ws;
  const int64_t stride = P.B * P.nc * P.M;
  ws[i] = prod;           // P: product of the chunk's multipliers
  ws[stride + i] = h;     // E: local end state
}

template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_chunk_carry(const LscanParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.M) return;
  const int64_t m = i % P.M, b = i / P.M;
  Chain<CT> ch{P, b, m};
  CT *ws = (CT *)P.ws;
  const int64_t stride = P.B * P.nc * P.M;
  CT hin = ch.h0();
  for (int cj = 0; cj < P.nc; ++cj) {
    const int64_t k = (b * P.nc + cj) * P.M + m;
    ws[2 * stride + k] = hin;  // state entering chunk cj
    hin = fma(ws[k], hin, ws[stride + k]);
  }
}

template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_chunk_fix(const LscanParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.nc * P.M) return;
  const int64_t m = i % P.M, cj = (i / P.M) % P.nc, b = i / (P.M * P.nc);
  Chain<CT> ch{P, b, m};
  const CT hin = ((const CT *)P.ws)[2 * P.B * P.nc * P.M + i];
  CT prod = 1;
  const int p0 = (int)cj * P.chunk;
  for (int pos = p0; pos < p0 + P.chunk && pos < (int)P.L; ++pos) {
    prod *= ch.mult(pos);
    const int64_t o = ch.h_off(ch.t_of(pos));
    vstore<CT>(P.h, o, fma(prod, hin, vload<CT>(P.h, o)));
  }
}

// ------------------------------------------------------------------ adjoint epilogue
// da_t = lambda_t * h_prev(t), dh0 = a_first * lambda_first (first in the forward's order).
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_grad(const LscanGradParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.L * P.M) return;
  const int64_t m = i % P.M, t = (i / P.M) % P.L, b = i / (P.M * P.L);
  const CT lam = vload<CT>(P.db, b * P.db.s0 + t * P.db.s1 + m * P.db.s2);
  const int64_t tp = P.reverse ? t + 1 : t - 1;  // previous step of the forward scan
  CT hp;
  if (tp >= 0 && tp < P.L) hp = vload<CT>(P.h, b * P.h.s0 + tp * P.h.s1 + m * P.h.s2);
  else hp = P.h0.p ? vload<CT>(P.h0, b * P.h0.s0 + m * P.h0.s1) : (CT)0;
  vstore<CT>(P.da, b * P.da.s0 + t * P.da.s1 + m * P.da.s2, lam * hp);
  const int64_t tfirst = P.reverse ? P.L - 1 : 0;
  if (t == tfirst && P.dh0.p)
    vstore<CT>(P.dh0, b * P.dh0.s0 + m * P.dh0.s1,
               vload<CT>(P.a, b * P.a.s0 + t * P.a.s1 + m * P.a.s2) * lam);
}

template <typename CT>
static hipError_t launch_lscan_t(const LscanParams &P, int algo, hipStream_t s) {
  const int64_t chains = P.B * P.M;
  switch (algo) {
    case 1:
      hipLaunchKernelGGL((k_lscan_seq<CT>), dim3((unsigned)((chains + 255) / 256)), dim3(256), 0, s, P);
      break;
    case 2:
      hipLaunchKernelGGL((k_lscan_hs<CT>), dim3((unsigned)P.M, (unsigned)P.B), dim3(256), 0, s, P);
      break;
    case 3:
      hipLaunchKernelGGL((k_lscan_bl<CT>), dim3((unsigned)P.M, (unsigned)P.B), dim3(256), 0, s, P);
      break;
    default: {
      const int64_t n = P.B * P.nc * P.M;
      hipLaunchKernelGGL((k_lscan_chunk_local<CT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, P);
      hipLaunchKernelGGL((k_lscan_chunk_carry<CT>), dim3((unsigned)((chains + 255) / 256)), dim3(256), 0, s, P);
      hipLaunchKernelGGL((k_lscan_chunk_fix<CT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, P);
    }
  }
  return hipGetLastError();
}

hipError_t launch_lscan(const LscanParams &P, int algo, int dtype, hipStream_t s) {
  return dtype == 3 ? launch_lscan_t<double>(P, algo, s) : launch_lscan_t<float>(P, algo, s);
}

hipError_t launch_lscan_grad(const LscanGradParams &P, int dtype, hipStream_t s) {
  const int64_t n = P.B * P.L * P.M;
  dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == 3) hipLaunchKernelGGL((k_lscan_grad<double>), grid, dim3(256), 0, s, P);
  else hipLaunchKernelGGL((k_lscan_grad<float>), grid, dim3(256), 0, s, P);
  return hipGetLastError();
}

}  // namespace ssm
