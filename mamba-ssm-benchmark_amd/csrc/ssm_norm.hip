// RMSNorm over the last dimension for gfx950: the LM's pre-norms (models/common.py:8-16,
// used at models/lm.py:63,95 and applied at :83,128).
//   y = (x r) w,  r = 1 / sqrt(mean_j x_j^2 + eps)  per row.
// Backward (g = dy w, xhat = x r):
//   dx = r (g - xhat mean_j(g xhat)),   dw = sum over rows of dy xhat.
// A wavefront owns whole rows: lane l holds columns l, l + 64, ... (coalesced 256-byte row
// segments) and the row sums are wavefront reductions whose result every lane holds bit for
// bit.  The backward issues all of a wavefront's row reads before its arithmetic and sums the
// weight gradient per workgroup (its wavefronts in order) into partials that a second kernel
// adds in workgroup order: no float atomics, bitwise reproducible.
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_wave.hpp"

namespace ssm {

template <typename T, int KC>
__global__ void __launch_bounds__(kNormThreads) k_norm_fwd(const NormParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kNormWaves + threadIdx.x / kWave;
  if (row >= p.R) return;  // uniform per wavefront
  const int C = (int)p.C;
  const T *xr = (const T *)p.x + row * p.sx;
  const T *w = (const T *)p.w;
  T v[KC];
  T ss = 0;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int j = lane + k * kWave;
    v[k] = j < C ? xr[j] : (T)0;
    ss = fma(v[k], v[k], ss);
  }
  ss = group_sum<kWave>(ss);
  const T r = (T)1 / sqrt(ss / (T)C + (T)p.eps);
  if (lane == 0) ((T *)p.rstd)[row] = r;
  T *yr = (T *)p.y + row * p.sy;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int j = lane + k * kWave;
    if (j < C) yr[j] = (v[k] * r) * w[j];  // the reference's order: (x r), then * w
  }
}

template <typename T, int KC, int RPW>
__global__ void __launch_bounds__(kNormThreads) k_norm_bwd(const NormParams p) {
  __shared__ T red[kNormWaves][KC * kWave];
  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  const int C = (int)p.C;
  const int64_t r0 = ((int64_t)blockIdx.x * kNormWaves + wv) * RPW;
  const T *w = (const T *)p.w;
  T wk[KC], acc[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int j = lane + k * kWave;
    wk[k] = j < C ? w[j] : (T)0;
    acc[k] = 0;
  }
  // every row's reads first; rows past the end re-read the last row and are not used
  T xv[RPW][KC], dv[RPW][KC], rs[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int64_t row = r0 + i < p.R ? r0 + i : p.R - 1;
    rs[i] = ((const T *)p.rstd)[row];
    const T *xr = (const T *)p.x + row * p.sx, *dr = (const T *)p.dy + row * p.sdy;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int j = lane + k * kWave;
      xv[i][k] = j < C ? xr[j] : (T)0;
      dv[i][k] = j < C ? dr[j] : (T)0;
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    if (r0 + i >= p.R) break;  // uniform per wavefront
    const T r = rs[i];
    T dot = 0;
#pragma unroll
    for (int k = 0; k < KC; ++k) dot = fma(dv[i][k] * wk[k], xv[i][k] * r, dot);
    const T c = group_sum<kWave>(dot) / (T)C;
    T *dxr = (T *)p.dx + (r0 + i) * p.sdx;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int j = lane + k * kWave;
      const T xh = xv[i][k] * r;
      if (j < C) dxr[j] = r * (dv[i][k] * wk[k] - xh * c);
      acc[k] = fma(dv[i][k], xh, acc[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < KC; ++k) red[wv][k * kWave + lane] = acc[k];
  __syncthreads();
  for (int j = threadIdx.x; j < C; j += kNormThreads) {
    T s = 0;
#pragma unroll
    for (int q = 0; q < kNormWaves; ++q) s += red[q][j];
    ((T *)p.ws)[(int64_t)blockIdx.x * C + j] = s;
  }
}

// dw_j = sum over the backward's workgroups (in order) of their partials: a workgroup of
// kNormFinThreads lanes per 64 columns, kNormFinThreads / 64 lanes per column each summing
// a contiguous range of partials, then those ranges in order.
template <typename T>
__global__ void __launch_bounds__(kNormFinThreads) k_norm_fin(const NormParams p) {
  constexpr int Q = kNormFinThreads / kWave;
  __shared__ T part[Q][kWave];
  const int lane = threadIdx.x % kWave, q = threadIdx.x / kWave;
  const int64_t j = (int64_t)blockIdx.x * kWave + lane;
  const int64_t per = (p.nblk + Q - 1) / Q;
  const int64_t b0 = q * per, b1 = b0 + per < p.nblk ? b0 + per : p.nblk;
  T s = 0;
  if (j < p.C) {
    const T *src = (const T *)p.ws + j;
    int64_t b = b0;
    for (; b + 4 <= b1; b += 4) {  // four partials' reads issued together, added in order
      const T v0 = src[b * p.C], v1 = src[(b + 1) * p.C], v2 = src[(b + 2) * p.C], v3 = src[(b + 3) * p.C];
      s += v0;
      s += v1;
      s += v2;
      s += v3;
    }
    for (; b < b1; ++b) s += src[b * p.C];
  }
  part[q][lane] = s;
  __syncthreads();
  if (q == 0 && j < p.C) {
    T t = 0;
#pragma unroll
    for (int k = 0; k < Q; ++k) t += part[k][lane];
    ((T *)p.dw)[j] = t;
  }
}

template <typename T, int KC>
static hipError_t norm_launch(const NormParams &p, bool bwd, hipStream_t s) {
  if (!bwd) {
    hipLaunchKernelGGL((k_norm_fwd<T, KC>), dim3((unsigned)((p.R + kNormWaves - 1) / kNormWaves)),
                       dim3(kNormThreads), 0, s, p);
    return hipGetLastError();
  }
  constexpr int RPW = norm_rows_per_wave(KC);
  if (p.rpw != RPW) return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_norm_bwd<T, KC, RPW>), dim3((unsigned)p.nblk), dim3(kNormThreads), 0, s, p);
  hipLaunchKernelGGL((k_norm_fin<T>), dim3((unsigned)((p.C + kWave - 1) / kWave)), dim3(kNormFinThreads), 0, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t norm_kc(const NormParams &p, bool bwd, hipStream_t s) {
  switch (norm_kc_of(p.C)) {
    case 1: return norm_launch<T, 1>(p, bwd, s);
    case 2: return norm_launch<T, 2>(p, bwd, s);
    case 4: return norm_launch<T, 4>(p, bwd, s);
    case 8: return norm_launch<T, 8>(p, bwd, s);
    case 16: return norm_launch<T, 16>(p, bwd, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_norm(const NormParams &p, int dtype, bool bwd, hipStream_t s) {
  return dtype == 3 ? norm_kc<double>(p, bwd, s) : norm_kc<float>(p, bwd, s);
}

}  // namespace ssm
