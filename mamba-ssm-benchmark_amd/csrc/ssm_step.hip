// Single-token recurrent step (decode) for gfx950.
//
// Replaces the inline decode of models/mamba.py:113-118 (discretize at L = 1, h = a h0 + b,
// y = einsum("bdn,bn->bd")) and the state write-back of :122-123, with the D skip and gate of
// :124 fused.  One lane per (channel, state) as in the fused scan; the state is updated in
// place and the sum over states is a butterfly of cross-lane adds inside each NP-lane group.
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"

namespace ssm {

template <typename IT, int NP, int METHOD>
__global__ void __launch_bounds__(kThreads) k_step(const StepParams p) {
  typedef typename Conv<IT>::CT CT;
  constexpr int DT = kThreads / NP;
  const int tid = threadIdx.x;
  const int c = tid / NP, n = tid % NP;
  const int64_t b = blockIdx.y;
  const int64_t d = (int64_t)blockIdx.x * DT + c;
  const bool dval = d < p.D, nval = n < p.N;
  CT y = 0, xv = 0;
  if (dval) {
    xv = Conv<IT>::load(vp<IT>(p.x) + b * p.x.s0 + d * p.x.s1);
    CT dt = Conv<IT>::load(vp<IT>(p.dt) + b * p.dt.s0 + d * p.dt.s1);
    if (p.has_bias) dt += vload<CT>(p.bias, d * p.bias.s0);
    if (p.softplus) dt = softplus_ct<CT>(dt);
    if (nval) {
      const AConst<CT> ac = make_aconst(vload<CT>(p.A, d * p.A.s0 + n * p.A.s1));
      CT a, coef;
      if constexpr (METHOD == 0) disc_zoh_m1(dt, ac, a, coef);  // a holds a - 1
      else disc<METHOD>(dt, ac, a, coef);
      const CT Bv = Conv<IT>::load(vp<IT>(p.Bm) + b * p.Bm.s0 + n * p.Bm.s1);
      const CT Cv = Conv<IT>::load(vp<IT>(p.Cm) + b * p.Cm.s0 + n * p.Cm.s1);
      const int64_t ho = b * p.h.s0 + d * p.h.s1 + n * p.h.s2;
      CT h = vload<CT>(p.h, ho);
      const CT bx = bcoef<METHOD>(dt, coef) * (Bv * xv);
      h = METHOD == 0 ? fma(a, h, h + bx) : fma(a, h, bx);
      vstore<CT>(p.h, ho, h);
      y = Cv * h;
    }
  }
#pragma unroll
  for (int off = NP / 2; off > 0; off >>= 1) y += __shfl_xor(y, off);
  if (n == 0 && dval) {
    CT o = y;
    if (p.has_D) o += vload<CT>(p.Dsk, d * p.Dsk.s0) * xv;
    if (p.has_z) {
      const CT zv = Conv<IT>::load(vp<IT>(p.z) + b * p.z.s0 + d * p.z.s1);
      o *= zv * sigmoid_ct<CT>(zv);
    }
    Conv<IT>::store(vpw<IT>(p.out) + b * p.out.s0 + d * p.out.s1, o);
  }
}

template <typename IT, int NP, int M>
static hipError_t launch_step_t(const StepParams &p, hipStream_t s) {
  constexpr int DT = kThreads / NP;
  dim3 grid((unsigned)((p.D + DT - 1) / DT), (unsigned)p.B);
  hipLaunchKernelGGL((k_step<IT, NP, M>), grid, dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

template <typename IT, int NP>
static hipError_t launch_step_m(const StepParams &p, int method, hipStream_t s) {
  switch (method) {
    case 0: return launch_step_t<IT, NP, 0>(p, s);
    case 1: return launch_step_t<IT, NP, 1>(p, s);
    default: return launch_step_t<IT, NP, 2>(p, s);
  }
}

template <typename IT>
static hipError_t launch_step_n(const StepParams &p, int method, int np, hipStream_t s) {
  switch (np) {
    case 8: return launch_step_m<IT, 8>(p, method, s);
    case 16: return launch_step_m<IT, 16>(p, method, s);
    case 32: return launch_step_m<IT, 32>(p, method, s);
    default: return launch_step_m<IT, 64>(p, method, s);
  }
}

hipError_t launch_step(const StepParams &p, int dtype, int method, int np, hipStream_t s) {
  switch (dtype) {
    case 0: return launch_step_n<float>(p, method, np, s);
    case 1: return launch_step_n<bf16_t>(p, method, np, s);
    case 2: return launch_step_n<f16_t>(p, method, np, s);
    default: return launch_step_n<double>(p, method, np, s);
  }
}

}  // namespace ssm
