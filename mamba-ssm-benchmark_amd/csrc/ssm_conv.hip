// Causal depthwise conv1d (+ SiLU) for gfx950: the producer of the scan's input in the Mamba
// block, models/mamba.py:101-107:
//   xc = pad_left(x, W-1) (or [state, x]);  out = silu(conv1d(xc, w, bias, groups=D));
//   state <- the last W-1 columns of xc.
// x and out are (B, L, D) views (the in_proj split of models/mamba.py:100 is D-contiguous),
// read and written with lanes along D.  One lane owns (b, d, a block of TB steps) and slides a
// register window of the W-1 previous inputs; the block's first window comes from the inputs
// before it (or from the carried state / zeros at t = 0).  The backward recomputes the conv
// output for the SiLU derivative, forms dx with the transposed taps, and writes per-block
// partial sums of dweight / dbias that a second kernel adds in a fixed order.
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"

namespace ssm {

template <typename CT>
__device__ __forceinline__ CT silu_ct(CT v) {
  return v * sigmoid_ct<CT>(v);
}

template <typename IT, int W>
__global__ void __launch_bounds__(kThreads) k_conv_fwd(const ConvParams p) {
  typedef typename Conv<IT>::CT CT;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= p.B * p.D * p.nblk) return;
  const int64_t d = i % p.D, blk = (i / p.D) % p.nblk, b = i / (p.D * p.nblk);
  const int L = (int)p.L;
  const int t0 = (int)blk * p.TB, t1 = t0 + p.TB < L ? t0 + p.TB : L;
  const IT *xb = vp<IT>(p.x) + b * p.x.s0 + d * p.x.s2;
  CT w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = vload<CT>(p.w, d * p.w.s0 + j * p.w.s1);
  const CT bias = p.has_bias ? vload<CT>(p.bias, d * p.bias.s0) : (CT)0;
  // win[j] = input at time t - (W-1) + j for the next output t
  CT win[W > 1 ? W - 1 : 1];
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const int s = t0 - (W - 1) + j;
    if (s >= 0) win[j] = Conv<IT>::load(xb + (int64_t)s * p.x.s1);
    else win[j] = p.has_sin ? Conv<IT>::load(vp<IT>(p.sin) + b * p.sin.s0 + d * p.sin.s1 + (W - 1 + s) * p.sin.s2) : (CT)0;
  }
  if (p.has_sout && blk == 0) {
    // the new state: inputs L-(W-1) .. L-1 of [state, x]; written by the block that reads the
    // old state, so an in-place update (sout == sin) is safe
#pragma unroll
    for (int j = 0; j < W - 1; ++j) {
      const int s = L - (W - 1) + j;
      CT v;
      if (s >= 0) v = Conv<IT>::load(xb + (int64_t)s * p.x.s1);
      else v = p.has_sin ? Conv<IT>::load(vp<IT>(p.sin) + b * p.sin.s0 + d * p.sin.s1 + (W - 1 + s) * p.sin.s2) : (CT)0;
      Conv<IT>::store(vpw<IT>(p.sout) + b * p.sout.s0 + d * p.sout.s1 + j * p.sout.s2, v);
    }
  }
  IT *ob = vpw<IT>(p.out) + b * p.out.s0 + d * p.out.s2;
  for (int t = t0; t < t1; ++t) {
    const CT xv = Conv<IT>::load(xb + (int64_t)t * p.x.s1);
    CT acc = fma(w[W - 1], xv, bias);
#pragma unroll
    for (int j = 0; j < W - 1; ++j) acc = fma(w[j], win[j], acc);
#pragma unroll
    for (int j = 0; j + 1 < W - 1; ++j) win[j] = win[j + 1];
    if constexpr (W > 1) win[W - 2] = xv;
    Conv<IT>::store(ob + (int64_t)t * p.out.s1, p.silu ? silu_ct(acc) : acc);
  }
}

template <typename IT, int W>
__global__ void __launch_bounds__(kThreads) k_conv_bwd(const ConvParams p) {
  typedef typename Conv<IT>::CT CT;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= p.B * p.D * p.nblk) return;
  const int64_t d = i % p.D, blk = (i / p.D) % p.nblk, b = i / (p.D * p.nblk);
  const int L = (int)p.L;
  const int t0 = (int)blk * p.TB, t1 = t0 + p.TB < L ? t0 + p.TB : L;
  const IT *xb = vp<IT>(p.x) + b * p.x.s0 + d * p.x.s2;
  const IT *gb = vp<IT>(p.dout) + b * p.dout.s0 + d * p.dout.s2;
  IT *dxb = vpw<IT>(p.dx) + b * p.dx.s0 + d * p.dx.s2;
  CT w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = vload<CT>(p.w, d * p.w.s0 + j * p.w.s1);
  const CT bias = p.has_bias ? vload<CT>(p.bias, d * p.bias.s0) : (CT)0;
  auto xat = [&](int s) -> CT {  // input at time s of [state, x]
    if (s >= 0) return s < L ? Conv<IT>::load(xb + (int64_t)s * p.x.s1) : (CT)0;
    return p.has_sin ? Conv<IT>::load(vp<IT>(p.sin) + b * p.sin.s0 + d * p.sin.s1 + (W - 1 + s) * p.sin.s2) : (CT)0;
  };
  // xw[j]: input at time t' - (W-1) + j for the conv output at t'; gw[j]: g at time t' - j
  CT xw[W > 1 ? W - 1 : 1], gw[W];
#pragma unroll
  for (int j = 0; j < W - 1; ++j) xw[j] = xat(t0 - (W - 1) + j);
#pragma unroll
  for (int j = 0; j < W; ++j) gw[j] = 0;
  CT dwp[W], dbp = 0;
#pragma unroll
  for (int j = 0; j < W; ++j) dwp[j] = 0;
  const int tend = t1 + W - 1 < L ? t1 + W - 1 : L;  // g is needed up to t1 + W - 2
  for (int tp = t0; tp < t1 + W - 1; ++tp) {
    CT g = 0, xv = 0;
    if (tp < tend) {
      xv = Conv<IT>::load(xb + (int64_t)tp * p.x.s1);
      CT pre = fma(w[W - 1], xv, bias);
#pragma unroll
      for (int j = 0; j < W - 1; ++j) pre = fma(w[j], xw[j], pre);
      g = Conv<IT>::load(gb + (int64_t)tp * p.dout.s1);
      if (p.silu) {
        const CT sg = sigmoid_ct<CT>(pre);
        g *= sg * ((CT)1 + pre * ((CT)1 - sg));
      }
      if (tp < t1) {  // this block's own steps feed dweight / dbias
#pragma unroll
        for (int j = 0; j < W - 1; ++j) dwp[j] = fma(g, xw[j], dwp[j]);
        dwp[W - 1] = fma(g, xv, dwp[W - 1]);
        dbp += g;
      }
    }
#pragma unroll
    for (int j = W - 1; j > 0; --j) gw[j] = gw[j - 1];
    gw[0] = g;
#pragma unroll
    for (int j = 0; j + 1 < W - 1; ++j) xw[j] = xw[j + 1];
    if constexpr (W > 1) xw[W - 2] = xv;
    const int t = tp - (W - 1);  // dx[t] = sum_j w[j] g[t + W-1 - j] = sum_j w[j] gw[j]
    if (t >= t0) {
      CT acc = 0;
#pragma unroll
      for (int j = 0; j < W; ++j) acc = fma(w[j], gw[j], acc);
      Conv<IT>::store(dxb + (int64_t)t * p.dx.s1, acc);
    }
  }
  CT *ws = (CT *)p.ws;
  const int64_t row = b * p.nblk + blk;
#pragma unroll
  for (int j = 0; j < W; ++j) ws[(row * p.D + d) * (W + 1) + j] = dwp[j];
  ws[(row * p.D + d) * (W + 1) + W] = dbp;
}

template <typename CT>
__global__ void __launch_bounds__(kThreads) k_conv_fin(const ConvParams p) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int W = (int)p.W;
  if (i >= p.D * (W + 1)) return;
  const int64_t d = i / (W + 1);
  const int j = (int)(i % (W + 1));
  const CT *ws = (const CT *)p.ws;
  CT s = 0;
  for (int64_t r = 0; r < p.B * p.nblk; ++r) s += ws[(r * p.D + d) * (W + 1) + j];
  if (j < W) vstore<CT>(p.dw, d * p.dw.s0 + j * p.dw.s1, s);
  else if (p.has_dbias) vstore<CT>(p.dbias, d * p.dbias.s0, s);
}

template <typename IT, int W>
static hipError_t conv_t(const ConvParams &p, bool bwd, hipStream_t s) {
  typedef typename Conv<IT>::CT CT;
  const int64_t n = p.B * p.D * p.nblk;
  const dim3 grid((unsigned)((n + kThreads - 1) / kThreads));
  if (!bwd) {
    hipLaunchKernelGGL((k_conv_fwd<IT, W>), grid, dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((k_conv_bwd<IT, W>), grid, dim3(kThreads), 0, s, p);
    const int64_t m = p.D * (W + 1);
    hipLaunchKernelGGL((k_conv_fin<CT>), dim3((unsigned)((m + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, p);
  }
  return hipGetLastError();
}

template <typename IT>
static hipError_t conv_w(const ConvParams &p, bool bwd, hipStream_t s) {
  switch (p.W) {
    case 1: return conv_t<IT, 1>(p, bwd, s);
    case 2: return conv_t<IT, 2>(p, bwd, s);
    case 3: return conv_t<IT, 3>(p, bwd, s);
    case 4: return conv_t<IT, 4>(p, bwd, s);
    case 5: return conv_t<IT, 5>(p, bwd, s);
    case 6: return conv_t<IT, 6>(p, bwd, s);
    case 7: return conv_t<IT, 7>(p, bwd, s);
    default: return conv_t<IT, 8>(p, bwd, s);
  }
}

hipError_t launch_conv(const ConvParams &p, int dtype, bool bwd, hipStream_t s) {
  switch (dtype) {
    case 0: return conv_w<float>(p, bwd, s);
    case 1: return conv_w<bf16_t>(p, bwd, s);
    case 2: return conv_w<f16_t>(p, bwd, s);
    default: return conv_w<double>(p, bwd, s);
  }
}

}  // namespace ssm
