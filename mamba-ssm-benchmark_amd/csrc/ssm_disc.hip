// Materialized discretization (models/scan.py:39-55) and its backward, for the composed
// scan path (models/scan.py:202-255), which discretizes a channel tile into (B, L, d, N)
// tensors, scans them with a chosen algorithm, and maps the scan's gradients (da, db) back to
// (ddelta, dA, dBm, dx) through autograd (:249).
//
// Forward: one lane per output element; the (B, L, D, N) outputs are written contiguously.
// Backward: a workgroup owns 256/NP channels x NP states and walks a group of (b, l) rows,
// with the reads of the next kDiscAhead rows in flight during a row's arithmetic and stores.
//   ddelta, dx  (B, L, D)  sums over n: DPP row permutations inside each NP-lane group;
//   dBm (B, L, N)          sum over d: per-row LDS reduction over the tile's channels into a
//                          (row, tile, n) partial, then a fixed-order sum over tiles;
//   dA (D, N)              sum over (b, l): register accumulation over the group's rows into a
//                          (group, d, n) partial, then a fixed-order sum over groups.
// All sums run in a fixed order, so results are bitwise reproducible.
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"

namespace ssm {

// Time rows per lane and pass: their reads are all issued before the first store (a wave's
// read waits would otherwise also wait for its earlier stores).
constexpr int kDiscRows = 8;
// Backward rows in flight per lane ahead of the row being computed.
constexpr int kDiscAhead = 4;

template <typename CT, int METHOD>
__global__ void __launch_bounds__(kThreads) k_disc_fwd(const DiscParams p) {
  // grid: x over the D*N elements of a (b, t) row (32-bit index, contiguous outputs), y over
  // groups of kDiscRows time rows (striding), z over b (striding); the per-(d, n) constants
  // are formed once
  const int e = blockIdx.x * kThreads + threadIdx.x;
  const int DN = (int)(p.D * p.N);
  if (e >= DN) return;
  const int n = e % (int)p.N, d = e / (int)p.N;
  const int L = (int)p.L;
  const AConst<CT> ac = make_aconst(vload<CT>(p.A, d * p.A.s0 + n * p.A.s1));
  for (int64_t b = blockIdx.z; b < p.B; b += gridDim.z) {
    for (int t0 = blockIdx.y * kDiscRows; t0 < L; t0 += gridDim.y * kDiscRows) {
      CT dt[kDiscRows], xv[kDiscRows], Bv[kDiscRows];
#pragma unroll
      for (int k = 0; k < kDiscRows; ++k) {  // clamped rows past the end are read, not stored
        const int64_t t = min(t0 + k, L - 1);
        dt[k] = vload<CT>(p.delta, b * p.delta.s0 + t * p.delta.s1 + d * p.delta.s2);
        xv[k] = vload<CT>(p.x, b * p.x.s0 + t * p.x.s1 + d * p.x.s2);
        Bv[k] = vload<CT>(p.Bm, b * p.Bm.s0 + t * p.Bm.s1 + n * p.Bm.s2);
      }
#pragma unroll
      for (int k = 0; k < kDiscRows; ++k) {
        if (t0 + k >= L) break;
        CT a, coef;
        disc<METHOD>(dt[k], ac, a, coef);
        const int64_t i = (b * p.L + t0 + k) * DN + e;
        ((CT *)p.a)[i] = a;
        ((CT *)p.b)[i] = bcoef<METHOD>(dt[k], coef) * (Bv[k] * xv[k]);
      }
    }
  }
}

// The float forward with 16-byte stores: a lane owns 4 consecutive states (n .. n+3) of one
// channel (N a multiple of 4), so a store instruction writes 1 KB of an output row where a lane
// per element wrote 256 B: 4x the bytes behind each outstanding memory instruction of the
// write-dominated pass.  B's 4 values of a row arrive as one 16-byte read.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kDiscQuadGroups = 64;  // row groups in the grid's y dimension (each walks L / (64 x 8))

template <int METHOD>
__global__ void __launch_bounds__(kThreads) k_disc_fwd4(const DiscParams p) {
  const int e4 = blockIdx.x * kThreads + threadIdx.x;  // the lane's quad within a (b, t) row
  const int DN4 = (int)(p.D * p.N / 4), N4 = (int)(p.N / 4);
  if (e4 >= DN4) return;
  const int n0 = (e4 % N4) * 4, d = e4 / N4;
  const int L = (int)p.L;
  AConst<float> ac[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) ac[j] = make_aconst(vload<float>(p.A, d * p.A.s0 + (n0 + j) * p.A.s1));
  for (int64_t b = blockIdx.z; b < p.B; b += gridDim.z) {
    for (int t0 = blockIdx.y * kDiscRows; t0 < L; t0 += gridDim.y * kDiscRows) {
      float dt[kDiscRows], xv[kDiscRows];
      f32x4 Bv[kDiscRows];
#pragma unroll
      for (int k = 0; k < kDiscRows; ++k) {  // clamped rows past the end are read, not stored
        const int64_t t = min(t0 + k, L - 1);
        dt[k] = vload<float>(p.delta, b * p.delta.s0 + t * p.delta.s1 + d * p.delta.s2);
        xv[k] = vload<float>(p.x, b * p.x.s0 + t * p.x.s1 + d * p.x.s2);
        Bv[k] = *(const f32x4 *)((const float *)p.Bm.p + b * p.Bm.s0 + t * p.Bm.s1 + n0);
      }
#pragma unroll
      for (int k = 0; k < kDiscRows; ++k) {
        if (t0 + k >= L) break;
        f32x4 av, bv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float a, coef;
          disc<METHOD>(dt[k], ac[j], a, coef);
          av[j] = a;
          bv[j] = bcoef<METHOD>(dt[k], coef) * (Bv[k][j] * xv[k]);
        }
        const int64_t i = (b * p.L + t0 + k) * DN4 + e4;
        ((f32x4 *)p.a)[i] = av;
        ((f32x4 *)p.b)[i] = bv;
      }
    }
  }
}

template <typename CT, int NP, int METHOD>
__global__ void __launch_bounds__(kThreads) k_disc_bwd(const DiscParams p) {
  constexpr int DT = kThreads / NP;
  __shared__ CT red[2][DT][NP];  // double-buffered by row parity: one barrier per row
  const int tid = threadIdx.x, c = tid / NP, n = tid % NP;
  const int64_t tile = blockIdx.x, g = blockIdx.y;
  const int64_t d = tile * DT + c;
  const bool valid = d < p.D && n < p.N;
  const int64_t dc = valid ? d : 0, nc = valid ? n : 0;  // clamped: every read stays in bounds
  const int64_t R = p.B * p.L;
  const int64_t r0 = g * p.rows_per_group, r1 = r0 + p.rows_per_group < R ? r0 + p.rows_per_group : R;
  AConst<CT> ac = make_aconst<CT>(-1);
  if (valid) ac = make_aconst(vload<CT>(p.A, d * p.A.s0 + n * p.A.s1));
  // Addresses: a uniform row offset (advanced one row at a time) plus the lane's 32-bit
  // element offset (the host checks that every lane offset fits in 31 bits).
  const uint32_t ldel = (uint32_t)(dc * p.delta.s2), lx = (uint32_t)(dc * p.x.s2), lB = (uint32_t)(nc * p.Bm.s2);
  const uint32_t lg = (uint32_t)(dc * p.N + nc);
  const uint32_t ldd = (uint32_t)(dc * p.ddelta.s2), ldx = (uint32_t)(dc * p.dx.s2);
  const int64_t DN = p.D * p.N;
  struct Row { CT dt, x, B, ga, gb; };
  // row offsets of the next row to fetch (delta, x, Bm, and the (row, d, n) gradients)
  int64_t fr = r0, fb = r0 / p.L, ft = r0 - fb * p.L;
  int64_t odel = fb * p.delta.s0 + ft * p.delta.s1, ox = fb * p.x.s0 + ft * p.x.s1,
          oB = fb * p.Bm.s0 + ft * p.Bm.s1, og = r0 * DN;
  const CT *const del = (const CT *)p.delta.p, *const xs = (const CT *)p.x.p, *const Bs = (const CT *)p.Bm.p;
  const CT *const das = (const CT *)p.da, *const dbs = (const CT *)p.db;
  // Rows are fetched kDiscAhead ahead of the one being computed (a ring of registers, the
  // loop unrolled over it).  Past the group's last row the fetch repeats that row, so every
  // read stays in bounds.
  auto fetch_next = [&]() {
    Row v;
    v.dt = (del + odel)[ldel];
    v.x = (xs + ox)[lx];
    v.B = (Bs + oB)[lB];
    v.ga = (das + og)[lg];
    v.gb = (dbs + og)[lg];
    if (fr + 1 < r1) {
      ++fr;
      og += DN;
      if (++ft == p.L) {
        ft = 0;
        ++fb;
        odel += p.delta.s0 - (p.L - 1) * p.delta.s1;
        ox += p.x.s0 - (p.L - 1) * p.x.s1;
        oB += p.Bm.s0 - (p.L - 1) * p.Bm.s1;
      } else {
        odel += p.delta.s1;
        ox += p.x.s1;
        oB += p.Bm.s1;
      }
    }
    return v;
  };
  // row offsets of the row being stored
  int64_t sb = r0 / p.L, st = r0 - sb * p.L;
  int64_t odd = sb * p.ddelta.s0 + st * p.ddelta.s1, odx = sb * p.dx.s0 + st * p.dx.s1;
  CT *const dds = (CT *)p.ddelta.p, *const dxs = (CT *)p.dx.p;
  CT *wsB = (CT *)p.ws_dB + (r0 * p.dtiles + tile) * p.N;
  const int64_t wstep = p.dtiles * p.N;
  // dA sums one term per row over the group's rows (hundreds): each read-ahead group of rows is
  // summed in CT and folded into a float64 running sum, so the rounding does not grow with the
  // number of rows
  double gA = 0;
  CT gA4 = 0;
  auto row = [&](const Row &cur, int buf) {
    CT gd = 0, gx = 0, gB = 0;
    if (valid) {
      CT a, coef, dadz, dbdd, d2f;
      disc<METHOD>(cur.dt, ac, a, coef);
      dfactors<METHOD>(cur.dt, ac, a, coef, dadz, dbdd, d2f);
      const CT bx = cur.B * cur.x, gz = cur.ga * dadz, gbc = cur.gb * bcoef<METHOD>(cur.dt, coef);
      gd = fma(ac.A, gz, cur.gb * dbdd * bx);
      gA4 += fma(cur.dt, gz, cur.gb * d2f * bx);
      gx = gbc * cur.B;
      gB = gbc * cur.x;
    }
    gd = group_sum<NP>(gd);
    gx = group_sum<NP>(gx);
    if (n == 0 && d < p.D) {
      (dds + odd)[ldd] = gd;
      (dxs + odx)[ldx] = gx;
    }
    red[buf][c][n] = gB;
    __syncthreads();
    if (tid < NP) {  // dBm partial of (row, state): sum over the tile's DT channels in channel order
      CT sum = 0;
#pragma unroll
      for (int k = 0; k < DT; ++k) sum += red[buf][k][tid];
      if (tid < p.N) wsB[tid] = sum;
    }
    wsB += wstep;
    if (++st == p.L) {
      st = 0;
      odd += p.ddelta.s0 - (p.L - 1) * p.ddelta.s1;
      odx += p.dx.s0 - (p.L - 1) * p.dx.s1;
    } else {
      odd += p.ddelta.s1;
      odx += p.dx.s1;
    }
  };
  Row q[kDiscAhead];
#pragma unroll
  for (int k = 0; k < kDiscAhead; ++k) q[k] = fetch_next();
  for (int64_t r = r0; r < r1; r += kDiscAhead) {
#pragma unroll
    for (int k = 0; k < kDiscAhead; ++k) {
      if (r + k >= r1) break;  // uniform over the workgroup
      const Row cur = q[k];
      q[k] = fetch_next();
      row(cur, k & 1);
    }
    gA += (double)gA4;
    gA4 = 0;
  }
  if (valid) ((CT *)p.ws_dA)[(g * p.D + d) * p.N + n] = (CT)gA;
}

template <typename CT>
__global__ void __launch_bounds__(kThreads) k_disc_fin(const DiscParams p) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t nB = p.B * p.L * p.N, nA = p.D * p.N;
  if (i < nB) {
    const int64_t n = i % p.N, r = i / p.N, b = r / p.L, t = r % p.L;
    const CT s = ordered_sum<16>((const CT *)p.ws_dB + r * p.dtiles * p.N + n, p.N, p.dtiles);
    vstore<CT>(p.dBm, b * p.dBm.s0 + t * p.dBm.s1 + n * p.dBm.s2, s);
  } else if (i < nB + nA) {
    const int64_t j = i - nB, n = j % p.N, d = j / p.N;
    const double s = ordered_sum<16, CT, double>((const CT *)p.ws_dA + j, nA, p.ngroups);  // float64 sum
    vstore<CT>(p.dA, d * p.dA.s0 + n * p.dA.s1, (CT)s);
  }
}

template <typename CT, int M>
static hipError_t disc_fwd_t(const DiscParams &p, hipStream_t s) {
  const int64_t ty = (p.L + kDiscRows - 1) / kDiscRows;
  // 16-byte stores: float, N a multiple of 4, B contiguous along n with 16-byte aligned rows
  const bool quads = sizeof(CT) == 4 && p.N % 4 == 0 && p.Bm.s2 == 1 && p.Bm.s1 % 4 == 0 && p.Bm.s0 % 4 == 0 &&
                     (uintptr_t)p.Bm.p % 16 == 0 && (uintptr_t)p.a % 16 == 0 && (uintptr_t)p.b % 16 == 0;
  const int64_t lanes = quads ? p.D * p.N / 4 : p.D * p.N;
  // the 16-byte kernel walks several row groups per workgroup (fewer, longer wavefronts)
  const int64_t tymax = quads ? kDiscQuadGroups : 65535;
  const dim3 grid((unsigned)((lanes + kThreads - 1) / kThreads), (unsigned)(ty < tymax ? ty : tymax),
                  (unsigned)(p.B < 65535 ? p.B : 65535));
  if (quads) hipLaunchKernelGGL((k_disc_fwd4<M>), grid, dim3(kThreads), 0, s, p);
  else hipLaunchKernelGGL((k_disc_fwd<CT, M>), grid, dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

template <typename CT>
static hipError_t disc_fwd_m(const DiscParams &p, int method, hipStream_t s) {
  return method == 0 ? disc_fwd_t<CT, 0>(p, s) : method == 1 ? disc_fwd_t<CT, 1>(p, s) : disc_fwd_t<CT, 2>(p, s);
}

hipError_t launch_disc_fwd(const DiscParams &p, int dtype, int method, int, hipStream_t s) {
  return dtype == 3 ? disc_fwd_m<double>(p, method, s) : disc_fwd_m<float>(p, method, s);
}

template <typename CT, int NP, int M>
static hipError_t disc_bwd_t(const DiscParams &p, hipStream_t s) {
  hipLaunchKernelGGL((k_disc_bwd<CT, NP, M>), dim3((unsigned)p.dtiles, (unsigned)p.ngroups), dim3(kThreads), 0, s, p);
  const int64_t n = p.B * p.L * p.N + p.D * p.N;
  hipLaunchKernelGGL((k_disc_fin<CT>), dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

template <typename CT, int NP>
static hipError_t disc_bwd_m(const DiscParams &p, int method, hipStream_t s) {
  return method == 0 ? disc_bwd_t<CT, NP, 0>(p, s) : method == 1 ? disc_bwd_t<CT, NP, 1>(p, s)
                                                                : disc_bwd_t<CT, NP, 2>(p, s);
}

template <typename CT>
static hipError_t disc_bwd_n(const DiscParams &p, int method, int np, hipStream_t s) {
  switch (np) {
    case 8: return disc_bwd_m<CT, 8>(p, method, s);
    case 16: return disc_bwd_m<CT, 16>(p, method, s);
    case 32: return disc_bwd_m<CT, 32>(p, method, s);
    default: return disc_bwd_m<CT, 64>(p, method, s);
  }
}

hipError_t launch_disc_bwd(const DiscParams &p, int dtype, int method, int np, hipStream_t s) {
  return dtype == 3 ? disc_bwd_n<double>(p, method, np, s) : disc_bwd_n<float>(p, method, np, s);
}

}  // namespace ssm
