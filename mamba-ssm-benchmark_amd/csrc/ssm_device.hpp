// Device-side building blocks shared by the gfx950 selective-scan kernels.
//
// Numerics of the float32 path (the reference computes in float32 on the GPU,
// kernels/triton_scan.py:56-67):
//   * a = exp(z) is one v_exp_f32 on z*log2(e).
//   * expm1(z) for ZOH must keep full relative accuracy when |z| is small (a - 1 alone loses
//     ~ulp(1)/|z|), so for |z| < TAU_EM1 it is a degree-4 Taylor polynomial of e^z - 1
//     (truncation < 7e-7 relative); above it a - 1 is exact given a (Sterbenz) and the
//     relative error is < ulp/|z| < 7e-7.
//   * the ZOH dA term needs f(z) = d/dz[(e^z - 1)/z] = (z e^z - expm1 z)/z^2; for
//     |z| < TAU_F it is the Taylor series sum_k (k+1) z^k/(k+2)! to degree 5
//     (truncation < 3e-7 relative), otherwise (dt*a - coef)/A, which is the same quantity
//     because coef = expm1(z)/A.
// The float64 path uses the device math library's exp/expm1 and the series only where
// |z| < 1e-3 (as the fp64 oracle does).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssm {

// ------------------------------------------------------------------ element types
struct bf16_t {
  uint16_t bits;
};
typedef _Float16 f16_t;

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return __uint_as_float(((uint32_t)v.bits) << 16); }
__device__ __forceinline__ float to_f32(f16_t v) { return (float)v; }

template <typename T> struct Conv;
template <> struct Conv<float> {
  typedef float CT;
  __device__ __forceinline__ static float load(const float *p) { return *p; }
  __device__ __forceinline__ static void store(float *p, float v) { *p = v; }
};
template <> struct Conv<bf16_t> {
  typedef float CT;
  __device__ __forceinline__ static float load(const bf16_t *p) { return to_f32(*p); }
  __device__ __forceinline__ static void store(bf16_t *p, float v) {
    // round to nearest even; NaN stays NaN
    uint32_t u = __float_as_uint(v);
    uint16_t r;
    if ((u & 0x7fffffffu) > 0x7f800000u) r = 0x7fc0;
    else r = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    p->bits = r;
  }
};
template <> struct Conv<f16_t> {
  typedef float CT;
  __device__ __forceinline__ static float load(const f16_t *p) { return (float)*p; }
  __device__ __forceinline__ static void store(f16_t *p, float v) { *p = (f16_t)v; }
};
template <> struct Conv<double> {
  typedef double CT;
  __device__ __forceinline__ static double load(const double *p) { return *p; }
  __device__ __forceinline__ static void store(double *p, double v) { *p = v; }
};

// ------------------------------------------------------------------ math helpers
constexpr float LOG2E = 1.4426950408889634f;
constexpr float TAU_EM1 = 0.09f;   // switch between Taylor expm1 and exp - 1 (|z|)
constexpr float TAU_F = 0.3f;      // switch between Taylor f(z) and the closed form (|z|)

__device__ __forceinline__ float fast_exp2(float v) { return __builtin_amdgcn_exp2f(v); }
__device__ __forceinline__ float fast_rcp(float v) { return __builtin_amdgcn_rcpf(v); }

// Sum over aligned groups of NP lanes (NP a power of two, 8..64), every lane of a group
// receiving the same bits.  Float: DPP row permutations inside each 16-lane row (lane i ^ 1,
// i ^ 2, the mirrored quad of its half row, the mirrored half row), then cross-row shuffles.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int NP>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(NP >= 8 && NP <= 64 && (NP & (NP - 1)) == 0, "group size");
  v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  if constexpr (NP >= 16) v += dpp_f<0x140>(v);  // row_mirror
  if constexpr (NP >= 32) v += __shfl_xor(v, 16);
  if constexpr (NP >= 64) v += __shfl_xor(v, 32);
  return v;
}
template <int NP>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
  for (int off = NP / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// expm1 for z <= ~0 given z2 = z*log2(e) and a = 2^z2; Taylor in z2 with coefficients ln2^k/k!.
__device__ __forceinline__ float em1_from(float z2, float a) {
  const float c1 = 0.6931471805599453f, c2 = 0.2402265069591007f, c3 = 0.05550410866482158f,
              c4 = 0.009618129107628477f;
  float p = z2 * fmaf(z2, fmaf(z2, fmaf(z2, c4, c3), c2), c1);
  return (fabsf(z2) < TAU_EM1 * LOG2E) ? p : (a - 1.0f);
}

// f(z) = sum_k (k+1) z^k / (k+2)!, degree 5.
__device__ __forceinline__ float fseries(float z) {
  return fmaf(z, fmaf(z, fmaf(z, fmaf(z, fmaf(z, 1.0f / 840.0f, 1.0f / 144.0f), 1.0f / 30.0f), 0.125f),
                  1.0f / 3.0f), 0.5f);
}

// softplus(v) = max(v, 0) + log1p(w), w = exp(-|v|) in (0, 1], with log1p(w) = 2 atanh(s),
// s = w / (2 + w) <= 1/3, summed as 2 s (1 + s^2/3 + ... + s^14/15) (truncation < 2e-9 relative).
// Within 5 ulp of the exact value over all v (float32 emulation, worst-case rcp rounding); equals
// v for v > 20 like the thresholded softplus of the reference (models/mamba.py:76).
__device__ __forceinline__ float softplusf(float v) {
  const float w = __expf(-fabsf(v));
  const float s = w * fast_rcp(2.0f + w);
  const float t = s * s;
  float q = fmaf(t, 1.0f / 15.0f, 1.0f / 13.0f);
  q = fmaf(q, t, 1.0f / 11.0f);
  q = fmaf(q, t, 1.0f / 9.0f);
  q = fmaf(q, t, 1.0f / 7.0f);
  q = fmaf(q, t, 1.0f / 5.0f);
  q = fmaf(q, t, 1.0f / 3.0f);
  q = fmaf(q, t, 1.0f);
  return fmaxf(v, 0.0f) + 2.0f * s * q;
}
__device__ __forceinline__ double softplusd(double v) { return v > 20.0 ? v : log1p(exp(v)); }
__device__ __forceinline__ float sigmoidf(float v) { return fast_rcp(1.0f + __expf(-v)); }
__device__ __forceinline__ double sigmoidd(double v) { return 1.0 / (1.0 + exp(-v)); }

// Per-(d, n) constants of the discretization.
template <typename CT> struct AConst {
  CT A, A2, invA;
};

template <typename CT>
__device__ __forceinline__ AConst<CT> make_aconst(CT A) {
  AConst<CT> c;
  c.A = A;
  c.A2 = A * (CT)1.4426950408889634;
  c.invA = (CT)1 / A;
  return c;
}

// Discretize one (t, d, n) element:  a = exp(dt A) (or the Tustin ratio), and the
// coefficient `coef` with b = coef * B * x.  For bilinear, `coef` holds u = 1/(1 - z/2)
// (the backward needs u; b uses dt*u).
template <int METHOD>
__device__ __forceinline__ void disc(float dt, const AConst<float> &c, float &a, float &coef) {
  if (METHOD == 0) {
    float z2 = dt * c.A2;
    a = fast_exp2(z2);
    coef = em1_from(z2, a) * c.invA;
  } else if (METHOD == 1) {
    a = fast_exp2(dt * c.A2);
    coef = dt;
  } else {
    float hz = 0.5f * dt * c.A;
    float u = fast_rcp(1.0f - hz);
    a = (1.0f + hz) * u;
    coef = u;
  }
}

template <int METHOD>
__device__ __forceinline__ void disc(double dt, const AConst<double> &c, double &a, double &coef) {
  double z = dt * c.A;
  if (METHOD == 0) {
    a = exp(z);
    coef = expm1(z) * c.invA;
  } else if (METHOD == 1) {
    a = exp(z);
    coef = dt;
  } else {
    double u = 1.0 / (1.0 - 0.5 * z);
    a = (1.0 + 0.5 * z) * u;
    coef = u;
  }
}

// ZOH with a - 1 instead of a: am1 = expm1(dt A) (the accurate polynomial / a - 1 value above)
// and coef = am1 / A.  Carrying am1 lets a product a * v be formed as v + am1 * v, which keeps
// the relative accuracy of expm1 when a is close to 1.
__device__ __forceinline__ void disc_zoh_m1(float dt, const AConst<float> &c, float &am1, float &coef) {
  const float z2 = dt * c.A2;
  am1 = em1_from(z2, fast_exp2(z2));
  coef = am1 * c.invA;
}
__device__ __forceinline__ void disc_zoh_m1(double dt, const AConst<double> &c, double &am1, double &coef) {
  am1 = expm1(dt * c.A);
  coef = am1 * c.invA;
}
// a - 1 alone (ZOH)
__device__ __forceinline__ float zoh_am1(float dt, const AConst<float> &c) {
  const float z2 = dt * c.A2;
  return em1_from(z2, fast_exp2(z2));
}
__device__ __forceinline__ double zoh_am1(double dt, const AConst<double> &c) { return expm1(dt * c.A); }

// b coefficient multiplying B*x (bilinear stores u in coef).
template <int METHOD, typename CT>
__device__ __forceinline__ CT bcoef(CT dt, CT coef) {
  return METHOD == 2 ? dt * coef : coef;
}

// Backward per-element derivative factors (kernels/triton_scan.py:196-216):
//   dadz  = da/dz            (a for zoh/euler, u^2 for bilinear)
//   dbdd  = factor with db/ddelta = dbdd * B x   (a for zoh, 1 for euler, u^2 for bilinear)
//   d2f   = factor with db/dA     = d2f  * B x   (dt^2 f(z), 0, dt^2 u^2 / 2)
template <int METHOD>
__device__ __forceinline__ void dfactors(float dt, const AConst<float> &c, float a, float coef,
                                         float &dadz, float &dbdd, float &d2f) {
  if (METHOD == 0) {
    dadz = a;
    dbdd = a;
    float z = dt * c.A;
    float fs = fseries(z) * (dt * dt);
    float fd = fmaf(dt, a, -coef) * c.invA;
    d2f = (fabsf(z) < TAU_F) ? fs : fd;
  } else if (METHOD == 1) {
    dadz = a;
    dbdd = 1.0f;
    d2f = 0.0f;
  } else {
    float u2 = coef * coef;
    dadz = u2;
    dbdd = u2;
    d2f = 0.5f * dt * dt * u2;
  }
}

template <int METHOD>
__device__ __forceinline__ void dfactors(double dt, const AConst<double> &c, double a, double coef,
                                         double &dadz, double &dbdd, double &d2f) {
  if (METHOD == 0) {
    dadz = a;
    dbdd = a;
    double z = dt * c.A;
    if (fabs(z) < 1e-3) {
      d2f = (0.5 + z * (1.0 / 3.0 + z * (0.125 + z / 30.0))) * dt * dt;
    } else {
      d2f = (z * a - expm1(z)) / (z * z) * dt * dt;
    }
  } else if (METHOD == 1) {
    dadz = a;
    dbdd = 1.0;
    d2f = 0.0;
  } else {
    double u2 = coef * coef;
    dadz = u2;
    dbdd = u2;
    d2f = 0.5 * dt * dt * u2;
  }
}

template <typename CT> __device__ __forceinline__ CT softplus_ct(CT v);
template <> __device__ __forceinline__ float softplus_ct<float>(float v) { return softplusf(v); }
template <> __device__ __forceinline__ double softplus_ct<double>(double v) { return softplusd(v); }
template <typename CT> __device__ __forceinline__ CT sigmoid_ct(CT v);
template <> __device__ __forceinline__ float sigmoid_ct<float>(float v) { return sigmoidf(v); }
template <> __device__ __forceinline__ double sigmoid_ct<double>(double v) { return sigmoidd(v); }

}  // namespace ssm
