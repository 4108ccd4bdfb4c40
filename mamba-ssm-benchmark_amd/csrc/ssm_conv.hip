// Causal depthwise conv1d (+ SiLU) for gfx950: the producer of the scan's input in the Mamba
// block, models/mamba.py:101-107:
//   xc = pad_left(x, W-1) (or [state, x]);  out = silu(conv1d(xc, w, bias, groups=D));
//   state <- the last W-1 columns of xc.
// x and out are (B, L, D) views (the in_proj split of models/mamba.py:100 is D-contiguous).
// A workgroup covers 64 channels x 32 time steps; a lane owns one channel and kConvTT = 8
// consecutive steps, reads the W-1 inputs before them as well (neighbouring lanes along D make
// every read coalesced; the overlap between time blocks is served from cache), and all its
// reads are issued before any arithmetic, so the kernel is bound by HBM rather than by a chain
// of dependent loads.  Because kConvTT >= W-1, only a lane of the first time block reads the
// carried state, and that lane also writes the new state (after reading), so the update can
// be in place.  The backward recomputes the pre-activation for the SiLU derivative, forms dx
// with the transposed taps, and reduces dweight / dbias over the workgroup's 4 time blocks in
// LDS before writing one partial row per workgroup; a second kernel adds the rows in a fixed
// order.
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"

namespace ssm {

template <typename CT>
__device__ __forceinline__ CT silu_ct(CT v) {
  return v * sigmoid_ct<CT>(v);
}

constexpr int kConvThreads = kConvDG * kConvTG;

// input at time s of [state, x] for channel d of batch row b (0 past the end)
template <typename IT, int W>
__device__ __forceinline__ typename Conv<IT>::CT conv_in(const ConvParams &p, int64_t b, int64_t d, int s) {
  typedef typename Conv<IT>::CT CT;
  if (s >= 0) return s < (int)p.L ? Conv<IT>::load(vp<IT>(p.x) + b * p.x.s0 + (int64_t)s * p.x.s1 + d * p.x.s2) : (CT)0;
  if (!p.has_sin) return (CT)0;
  return Conv<IT>::load(vp<IT>(p.sin) + b * p.sin.s0 + d * p.sin.s1 + (int64_t)(W - 1 + s) * p.sin.s2);
}

template <typename IT, int W>
__global__ void __launch_bounds__(kConvThreads) k_conv_fwd(const ConvParams p) {
  typedef typename Conv<IT>::CT CT;
  constexpr int TT = kConvTT, NX = TT + W - 1;
  const int64_t d = (int64_t)blockIdx.x * kConvDG + threadIdx.x % kConvDG;
  const int t0 = ((int)blockIdx.y * kConvTG + (int)threadIdx.x / kConvDG) * TT;
  const int64_t b = blockIdx.z;
  const int L = (int)p.L;
  if (d >= p.D || t0 >= L) return;
  CT w[W], xin[NX];  // xin[k]: input at time t0 - (W-1) + k
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = vload<CT>(p.w, d * p.w.s0 + j * p.w.s1);
  const CT bias = p.has_bias ? vload<CT>(p.bias, d * p.bias.s0) : (CT)0;
#pragma unroll
  for (int k = 0; k < NX; ++k) xin[k] = conv_in<IT, W>(p, b, d, t0 - (W - 1) + k);
  if (p.has_sout && t0 == 0) {
    // the new state: inputs L-(W-1) .. L-1 of [state, x]; this lane is the only reader of the
    // old state, and it reads before it writes
    CT ns[W > 1 ? W - 1 : 1];
#pragma unroll
    for (int j = 0; j < W - 1; ++j) ns[j] = conv_in<IT, W>(p, b, d, L - (W - 1) + j);
#pragma unroll
    for (int j = 0; j < W - 1; ++j) Conv<IT>::store(vpw<IT>(p.sout) + b * p.sout.s0 + d * p.sout.s1 + j * p.sout.s2, ns[j]);
  }
  IT *ob = vpw<IT>(p.out) + b * p.out.s0 + d * p.out.s2;
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    CT acc = bias;
#pragma unroll
    for (int j = 0; j < W; ++j) acc = fma(w[j], xin[tt + j], acc);
    if (t0 + tt < L) Conv<IT>::store(ob + (int64_t)(t0 + tt) * p.out.s1, p.silu ? silu_ct(acc) : acc);
  }
}

template <typename IT, int W>
__global__ void __launch_bounds__(kConvThreads) k_conv_bwd(const ConvParams p) {
  typedef typename Conv<IT>::CT CT;
  constexpr int TT = kConvTT, NG = TT + W - 1, NX = TT + 2 * (W - 1);
  __shared__ CT red[kConvTG][W + 1][kConvDG];
  const int dl = threadIdx.x % kConvDG, tg = threadIdx.x / kConvDG;
  const int64_t d = (int64_t)blockIdx.x * kConvDG + dl;
  const int t0 = ((int)blockIdx.y * kConvTG + tg) * TT;
  const int64_t b = blockIdx.z;
  const int L = (int)p.L;
  const bool live = d < p.D && t0 < L;
  const int64_t dc = live ? d : 0;
  CT dwp[W + 1];  // dweight taps, then dbias
#pragma unroll
  for (int j = 0; j <= W; ++j) dwp[j] = 0;
  if (live) {
    CT w[W], xin[NX], g[NG];  // xin[k]: input at t0 - (W-1) + k; g[k]: dout x silu' at t0 + k
#pragma unroll
    for (int j = 0; j < W; ++j) w[j] = vload<CT>(p.w, dc * p.w.s0 + j * p.w.s1);
    const CT bias = p.has_bias ? vload<CT>(p.bias, dc * p.bias.s0) : (CT)0;
#pragma unroll
    for (int k = 0; k < NX; ++k) xin[k] = conv_in<IT, W>(p, b, dc, t0 - (W - 1) + k);
    const IT *gb = vp<IT>(p.dout) + b * p.dout.s0 + dc * p.dout.s2;
#pragma unroll
    for (int k = 0; k < NG; ++k)
      g[k] = t0 + k < L ? Conv<IT>::load(gb + (int64_t)(t0 + k) * p.dout.s1) : (CT)0;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      if (p.silu) {
        CT pre = bias;
#pragma unroll
        for (int j = 0; j < W; ++j) pre = fma(w[j], xin[k + j], pre);
        const CT sg = sigmoid_ct<CT>(pre);
        g[k] *= sg * ((CT)1 + pre * ((CT)1 - sg));
      }
    }
    IT *dxb = vpw<IT>(p.dx) + b * p.dx.s0 + dc * p.dx.s2;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      // dx[t] = sum_j w[j] g[t + W-1 - j]
      CT acc = 0;
#pragma unroll
      for (int j = 0; j < W; ++j) acc = fma(w[j], g[tt + W - 1 - j], acc);
      if (t0 + tt < L) {
        Conv<IT>::store(dxb + (int64_t)(t0 + tt) * p.dx.s1, acc);
#pragma unroll
        for (int j = 0; j < W; ++j) dwp[j] = fma(g[tt], xin[tt + j], dwp[j]);
        dwp[W] += g[tt];
      }
    }
  }
#pragma unroll
  for (int j = 0; j <= W; ++j) red[tg][j][dl] = dwp[j];
  __syncthreads();
  // one partial row per workgroup: the 4 time blocks in order
  const int64_t row = b * p.nblk + blockIdx.y;
  for (int e = threadIdx.x; e < (W + 1) * kConvDG; e += kConvThreads) {
    const int j = e / kConvDG, l = e % kConvDG;
    const int64_t dd = (int64_t)blockIdx.x * kConvDG + l;
    if (dd >= p.D) continue;
    CT sum = 0;
#pragma unroll
    for (int q = 0; q < kConvTG; ++q) sum += red[q][j][l];
    ((CT *)p.ws)[(row * p.D + dd) * (W + 1) + j] = sum;
  }
}

// dweight / dbias: the B * nblk partial rows summed in a fixed order.  A workgroup owns 64
// channels; its 16 row groups sum rows r = g, g + 16, ... (independent loads in flight), and
// the groups are added in order.
constexpr int kConvFinGroups = 16;

template <typename CT, int W>
__global__ void __launch_bounds__(kConvDG * kConvFinGroups) k_conv_fin(const ConvParams p) {
  __shared__ CT red[kConvFinGroups][W + 1][kConvDG];
  const int dl = threadIdx.x % kConvDG, g = threadIdx.x / kConvDG;
  const int64_t d = (int64_t)blockIdx.x * kConvDG + dl;
  const int64_t rows = p.B * p.nblk;
  const CT *ws = (const CT *)p.ws;
  CT acc[W + 1];
#pragma unroll
  for (int j = 0; j <= W; ++j) acc[j] = 0;
  if (d < p.D) {
#pragma unroll 4
    for (int64_t r = g; r < rows; r += kConvFinGroups) {
#pragma unroll
      for (int j = 0; j <= W; ++j) acc[j] += ws[(r * p.D + d) * (W + 1) + j];
    }
  }
#pragma unroll
  for (int j = 0; j <= W; ++j) red[g][j][dl] = acc[j];
  __syncthreads();
  for (int e = threadIdx.x; e < (W + 1) * kConvDG; e += kConvDG * kConvFinGroups) {
    const int j = e / kConvDG, l = e % kConvDG;
    const int64_t dd = (int64_t)blockIdx.x * kConvDG + l;
    if (dd >= p.D) continue;
    CT s = 0;
#pragma unroll
    for (int q = 0; q < kConvFinGroups; ++q) s += red[q][j][l];
    if (j < W) vstore<CT>(p.dw, dd * p.dw.s0 + j * p.dw.s1, s);
    else if (p.has_dbias) vstore<CT>(p.dbias, dd * p.dbias.s0, s);
  }
}

template <typename IT, int W>
static hipError_t conv_t(const ConvParams &p, bool bwd, hipStream_t s) {
  typedef typename Conv<IT>::CT CT;
  const dim3 grid((unsigned)((p.D + kConvDG - 1) / kConvDG), (unsigned)p.nblk, (unsigned)p.B);
  if (!bwd) {
    hipLaunchKernelGGL((k_conv_fwd<IT, W>), grid, dim3(kConvThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((k_conv_bwd<IT, W>), grid, dim3(kConvThreads), 0, s, p);
    hipLaunchKernelGGL((k_conv_fin<CT, W>), dim3(grid.x), dim3(kConvDG * kConvFinGroups), 0, s, p);
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
