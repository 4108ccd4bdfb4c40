/* float64 sequential selective scan and its adjoint -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the same arithmetic as oracle/scan_ref.py (selective_scan_fwd / _bwd) as a
 * per-channel C loop so that oracles for long sequences (L = 131072) finish in seconds:
 *   forward  : models/scan.py:264-274 (textbook loop) + gate models/mamba.py:124
 *   backward : kernels/triton_scan.py:171-226 (reverse adjoint walk, per-method terms)
 * Layouts are contiguous and logical: x, delta, z, out, y (B,L,D); A (D,N);
 * Bm, Cm (B,L,N); h0, last (B,D,N); Dskip (D).  Channels run in parallel with OpenMP;
 * dB/dC are accumulated per thread and summed in thread order (deterministic).
 * It is pinned against scan_ref.py by tests/test_oracle_kat.py (test_c_oracle_matches_numpy_oracle).
 * The backward optionally reports, per ddelta element, the sum over states of the magnitudes of
 * the terms it adds, per dA element the sum over batch and time and per dB and dC element the sum
 * over channels of its terms' magnitudes (the scale of the float32 rounding a kernel can leave in
 * that element).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define IDX3(b, l, d, L, D) (((int64_t)(b) * (L) + (l)) * (D) + (d))

static void disc(int method, double dt, double A, double Bx, double *a, double *b) {
  double z = dt * A;
  if (method == 0) {
    *a = exp(z);
    *b = expm1(z) / A * Bx;
  } else if (method == 1) {
    *a = exp(z);
    *b = dt * Bx;
  } else {
    double inv = 1.0 / (1.0 - 0.5 * z);
    *a = (1.0 + 0.5 * z) * inv;
    *b = dt * inv * Bx;
  }
}

static double silu(double v) { return v / (1.0 + exp(-v)); }

int ssm_oracle_fwd(int64_t B, int64_t L, int64_t D, int64_t N, int method, const double *x,
                   const double *delta, const double *A, const double *Bm, const double *Cm,
                   const double *h0, const double *Dskip, const double *z, double *out,
                   double *y, double *last, int nthreads) {
  if (method < 0 || method > 2) return 1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel for schedule(static)
  for (int64_t bd = 0; bd < B * D; ++bd) {
    int64_t b = bd / D, d = bd % D;
    double *h = (double *)malloc(sizeof(double) * N);
    for (int64_t n = 0; n < N; ++n) h[n] = h0 ? h0[(b * D + d) * N + n] : 0.0;
    for (int64_t t = 0; t < L; ++t) {
      double xv = x[IDX3(b, t, d, L, D)], dt = delta[IDX3(b, t, d, L, D)];
      double acc = 0.0;
      for (int64_t n = 0; n < N; ++n) {
        double a, bb;
        disc(method, dt, A[d * N + n], Bm[IDX3(b, t, n, L, N)] * xv, &a, &bb);
        h[n] = a * h[n] + bb;
        acc += Cm[IDX3(b, t, n, L, N)] * h[n];
      }
      if (y) y[IDX3(b, t, d, L, D)] = acc;
      double o = acc;
      if (Dskip) o += xv * Dskip[d];
      if (z) o *= silu(z[IDX3(b, t, d, L, D)]);
      out[IDX3(b, t, d, L, D)] = o;
    }
    if (last)
      for (int64_t n = 0; n < N; ++n) last[(b * D + d) * N + n] = h[n];
    free(h);
  }
  return 0;
}

int ssm_oracle_bwd(int64_t B, int64_t L, int64_t D, int64_t N, int method, const double *x,
                   const double *delta, const double *A, const double *Bm, const double *Cm,
                   const double *h0, const double *Dskip, const double *z, const double *dout,
                   const double *dlast, double *dx, double *ddelta, double *dA, double *dB,
                   double *dC, double *dD, double *dz, double *dh0, double *ddelta_mag, double *dA_mag,
                   double *dB_mag, double *dC_mag, int nthreads) {
  if (method < 0 || method > 2) return 1;
  int nt = 1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
  nt = omp_get_max_threads();
#endif
  int64_t BLN = B * L * N;
  double *pB = (double *)calloc((size_t)nt * BLN, sizeof(double));
  double *pC = (double *)calloc((size_t)nt * BLN, sizeof(double));
  double *pA = (double *)calloc((size_t)B * D * N, sizeof(double));
  double *pAm = (double *)calloc((size_t)B * D * N, sizeof(double));
  double *pBm = dB_mag ? (double *)calloc((size_t)nt * BLN, sizeof(double)) : NULL;
  double *pCm = dC_mag ? (double *)calloc((size_t)nt * BLN, sizeof(double)) : NULL;
  if (!pB || !pC || !pA || !pAm || (dB_mag && !pBm) || (dC_mag && !pCm)) {
    free(pB); free(pC); free(pA); free(pAm); free(pBm); free(pCm);
    return 2;
  }
#pragma omp parallel
  {
    int tid = 0;
#ifdef _OPENMP
    tid = omp_get_thread_num();
#endif
    double *myB = pB + (int64_t)tid * BLN, *myC = pC + (int64_t)tid * BLN;
    double *myBm = pBm ? pBm + (int64_t)tid * BLN : NULL, *myCm = pCm ? pCm + (int64_t)tid * BLN : NULL;
    double *hs = (double *)malloc(sizeof(double) * (L + 1) * N);
    double *dh = (double *)malloc(sizeof(double) * N);
#pragma omp for schedule(static)
    for (int64_t bd = 0; bd < B * D; ++bd) {
      int64_t b = bd / D, d = bd % D;
      /* forward recompute: hs[t+1] = h_t, hs[0] = h0 */
      for (int64_t n = 0; n < N; ++n) hs[n] = h0 ? h0[(b * D + d) * N + n] : 0.0;
      for (int64_t t = 0; t < L; ++t) {
        double xv = x[IDX3(b, t, d, L, D)], dt = delta[IDX3(b, t, d, L, D)];
        for (int64_t n = 0; n < N; ++n) {
          double a, bb;
          disc(method, dt, A[d * N + n], Bm[IDX3(b, t, n, L, N)] * xv, &a, &bb);
          hs[(t + 1) * N + n] = a * hs[t * N + n] + bb;
        }
      }
      for (int64_t n = 0; n < N; ++n) dh[n] = dlast ? dlast[(b * D + d) * N + n] : 0.0;
      for (int64_t t = L - 1; t >= 0; --t) {
        int64_t i3 = IDX3(b, t, d, L, D);
        double xv = x[i3], dt = delta[i3];
        double y = 0.0;
        for (int64_t n = 0; n < N; ++n) y += Cm[IDX3(b, t, n, L, N)] * hs[(t + 1) * N + n];
        double dyv = dout[i3];
        if (z) {
          double zz = z[i3], s = 1.0 / (1.0 + exp(-zz));
          double pre = y + (Dskip ? xv * Dskip[d] : 0.0);
          dz[i3] = dyv * pre * s * (1.0 + zz * (1.0 - s));
          dyv = dyv * zz * s;
        }
        double dxv = Dskip ? dyv * Dskip[d] : 0.0, ddt = 0.0, mag = 0.0;
        for (int64_t n = 0; n < N; ++n) {
          int64_t in = IDX3(b, t, n, L, N);
          double Av = A[d * N + n], Bv = Bm[in], h_t = hs[(t + 1) * N + n], hp = hs[t * N + n];
          myC[in] += dyv * h_t;
          if (myCm) myCm[in] += fabs(dyv * h_t);
          dh[n] += dyv * Cm[in];
          double zt = dt * Av, Bx = Bv * xv, da = dh[n] * hp, a, tA, tB;
          if (method == 0) {
            a = exp(zt);
            double e = expm1(zt), coef = e / Av, f;
            if (fabs(zt) < 1e-3) f = 0.5 + zt / 3.0 + zt * zt / 8.0 + zt * zt * zt / 30.0;
            else f = (zt * a - e) / (zt * zt);
            ddt += da * Av * a + dh[n] * a * Bx;
            mag += fabs(da * Av * a + dh[n] * a * Bx);
            tA = da * dt * a + dh[n] * dt * dt * f * Bx;
            tB = dh[n] * coef * xv;
            dxv += dh[n] * coef * Bv;
          } else if (method == 1) {
            a = exp(zt);
            ddt += da * Av * a + dh[n] * Bx;
            mag += fabs(da * Av * a + dh[n] * Bx);
            tA = da * dt * a;
            tB = dh[n] * dt * xv;
            dxv += dh[n] * dt * Bv;
          } else {
            double u = 1.0 / (1.0 - 0.5 * zt), u2 = u * u;
            a = (1.0 + 0.5 * zt) * u;
            ddt += da * Av * u2 + dh[n] * u2 * Bx;
            mag += fabs(da * Av * u2 + dh[n] * u2 * Bx);
            tA = da * dt * u2 + dh[n] * 0.5 * dt * dt * u2 * Bx;
            tB = dh[n] * dt * u * xv;
            dxv += dh[n] * dt * u * Bv;
          }
          pA[(b * D + d) * N + n] += tA;
          pAm[(b * D + d) * N + n] += fabs(tA);
          myB[in] += tB;
          if (myBm) myBm[in] += fabs(tB);
          dh[n] *= a;
        }
        dx[i3] = dxv;
        ddelta[i3] = ddt;
        if (ddelta_mag) ddelta_mag[i3] = mag;
      }
      if (dh0)
        for (int64_t n = 0; n < N; ++n) dh0[(b * D + d) * N + n] = dh[n];
    }
    free(hs);
    free(dh);
  }
  /* fixed-order reductions */
  for (int64_t i = 0; i < BLN; ++i) {
    double sb = 0.0, sc = 0.0;
    for (int k = 0; k < nt; ++k) { sb += pB[(int64_t)k * BLN + i]; sc += pC[(int64_t)k * BLN + i]; }
    dB[i] = sb;
    dC[i] = sc;
    if (dB_mag) {
      double sm = 0.0;
      for (int k = 0; k < nt; ++k) sm += pBm[(int64_t)k * BLN + i];
      dB_mag[i] = sm;
    }
    if (dC_mag) {
      double sm = 0.0;
      for (int k = 0; k < nt; ++k) sm += pCm[(int64_t)k * BLN + i];
      dC_mag[i] = sm;
    }
  }
  for (int64_t dn = 0; dn < D * N; ++dn) {
    double s = 0.0, m = 0.0;
    for (int64_t b = 0; b < B; ++b) s += pA[b * D * N + dn], m += pAm[b * D * N + dn];
    dA[dn] = s;
    if (dA_mag) dA_mag[dn] = m;
  }
  if (dD) {
    for (int64_t d = 0; d < D; ++d) dD[d] = 0.0;
    for (int64_t b = 0; b < B; ++b)
      for (int64_t t = 0; t < L; ++t)
        for (int64_t d = 0; d < D; ++d) {
          int64_t i3 = IDX3(b, t, d, L, D);
          double dyv = dout[i3];
          if (z) { double zz = z[i3]; dyv *= zz / (1.0 + exp(-zz)); }
          dD[d] += dyv * x[i3];
        }
  }
  free(pB);
  free(pC);
  free(pA);
  free(pAm);
  free(pBm);
  free(pCm);
  return 0;
}
