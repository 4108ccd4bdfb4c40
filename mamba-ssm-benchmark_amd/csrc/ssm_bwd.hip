// Fused selective-scan backward for gfx950.
//
// Replaces kernels/triton_scan.py:143-226 (_bwd_kernel) + :288-319 (host orchestration) and
// the backward of models/scan.py:219-255.  Same wavefront-private mapping as the forward (one
// lane per (channel, state), CW = 64/NP channels per wavefront), walking chunks of CK steps
// from the last to the first:
//   stage     x, delta (bias/softplus applied), dy = dout * silu(z), B, C into the wavefront's
//             LDS region; dz is produced here from the saved pre-gate output (per (t, d)).
//   recompute the chunk's states from the saved chunk-start state, keeping h_t, a_t and the
//             b-coefficient of all CK steps in VGPRs (no (B, L, D, N) buffer anywhere).
//   reverse   the adjoint recurrence dh_t = dy_t C_t + a_{t+1} dh_{t+1} (float64); per step each
//             lane forms its contributions to dx, ddelta (summed over the states inside the
//             wavefront) and dB, dC (summed over the wavefront's channels, then over the
//             workgroup's wavefronts with one workgroup barrier per chunk).  dA is accumulated
//             per lane in a VGPR over the whole sequence.
//   store     dx (+ D skip), ddelta (x sigmoid for softplus) with coalesced writes; per-tile
//             dB / dC partials to the workspace.
// The finalize kernel sums the dB / dC partials over channel tiles and dA / dD / d_bias over
// the batch, in a fixed order (bitwise reproducible; no float atomics).
#include "ssm_device.hpp"
#include "ssm_dpp.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"
#include "ssm_wave.hpp"

namespace ssm {

template <typename CT, int NP>
struct BwdWaveLds {
  static constexpr int CW = kWave / NP, CK = kCK, CKP = ck_pad((int)sizeof(CT)), RH = bwd_half();
  CT x[CW][CKP];
  CT dt[CW][CKP];
  CT dy[CW][CKP];
  CT sg[CW][CKP];
  CT gx[CW][CKP];
  CT gd[CW][CKP];
  CT B[NP][CKP];
  CT C[NP][CKP];
  CT pn[RH][CW][2][np_pad((int)sizeof(CT), NP)];  // (dx, ddelta) per-lane contributions, quantity-major
  CT pd[RH][CW][NP][2];  // (dB, dC) per-lane contributions
  CT lr[CK][lr_pad((int)sizeof(CT))];  // low-rank delta input rows of the chunk
  CT wr[CW][lr_pad((int)sizeof(CT))];  // low-rank weight rows of the wavefront's channels
};

template <typename CT, int NP, int WPB>
struct BwdShared {
  CT dbc[2][WPB][kCK][NP][2];  // per-wavefront (dB, dC) sums, double-buffered by chunk parity
};
template <typename CT, int NP>
struct BwdShared<CT, NP, 1> {};

template <typename IT, int NP, int METHOD, bool UL, bool LR>
__global__ void __launch_bounds__(kWave * bwd_waves(sizeof(typename Conv<IT>::CT), NP))
k_bwd(const BwdParams p) {
  typedef typename Conv<IT>::CT CT;
  typedef BwdWaveLds<CT, NP> WL;
  constexpr int CW = WL::CW, CK = WL::CK, RH = WL::RH;
  constexpr int WPB = bwd_waves(sizeof(CT), NP);
  constexpr int RB = 32 / (int)sizeof(CT) > RH ? RH : 32 / (int)sizeof(CT);  // register batch
  constexpr int NT = WPB * kWave;
  static_assert(sizeof(WL) == bwd_wave_bytes(sizeof(CT), NP), "LDS layout");
  static_assert(RH % RB == 0 && CK % RH == 0, "batches");
  __shared__ __align__(16) WL lds_all[WPB];
  __shared__ __align__(16) BwdShared<CT, NP, WPB> sh;

  const int tid = threadIdx.x;
  const int lane = tid % kWave, wv = tid / kWave;
  WL &S = lds_all[wv];
  const int c = lane / NP, n = lane % NP;
  const int64_t b = blockIdx.y;
  const int tile = blockIdx.x;
  const int dw = (tile * WPB + wv) * CW;
  const int d = dw + c;
  const bool dval = d < p.D, nval = n < p.N;
  const int L = (int)p.L, D = (int)p.D, N = (int)p.N;

  CT Av = (CT)-1;
  if (dval && nval) {
    Av = vload<CT>(p.A, d * p.A.s0 + n * p.A.s1);
    if (p.a_log) Av = -exp(Av);  // models/mamba.py:81
  }
  const AConst<CT> ac = make_aconst(Av);
  // The adjoint state is carried in float64: dh_t = a_{t+1} dh_{t+1} + dy_t C_t is a long,
  // slowly decaying accumulation (a -> 1 for small delta) and its float32 rounding dominates the
  // error of ddelta, which sums the state terms with cancellation.  One v_fma_f64 per step keeps
  // it at a single float64 rounding; dlast enters as "a_L dh_L" with a_L = 1.
  // For ZOH the recompute keeps am1 = a - 1 (accurate expm1) in aa[], and the step
  // a_{t+1} dh_{t+1} is formed as dh + am1 * dh in float64.
  constexpr bool M1 = METHOD == 0;
  double dh64 = 0.0;
  if (p.has_dlast && dval && nval)
    dh64 = (double)vload<CT>(p.dlast, b * p.dlast.s0 + d * p.dlast.s1 + n * p.dlast.s2);
  CT a_next = M1 ? (CT)0 : (CT)1;  // a (or a - 1 for ZOH) of the step after the current one
  CT h0v = 0;
  if (p.has_h0 && dval && nval) h0v = vload<CT>(p.h0, b * p.h0.s0 + d * p.h0.s1 + n * p.h0.s2);
  // dA from the per-state ddelta terms: a depends on dt and A only through z = dt A, and
  // b = g Bx with g = dt phi(z), so da/dA = (dt/A) da/ddt and dg/dA = (dt/A) dg/ddt - g/A.
  // Hence  A dA = sum_t [ dt pD_t - lambda_t b_t ],  pD_t = lambda_t (h_{t-1} da/ddt + db/ddt)
  // being this state's term of ddelta_t, for every discretization (no f(z) series needed).
  CT dA_acc = 0;

  const KView vx = p.x, vdt = with_layout<UL>(p.dt, p.x), vz = p.z;  // z keeps its own strides
  const KView vg = with_layout<UL>(p.dout, p.x);
  const KView vdz = p.dz;  // its own strides (e.g. the gate half of an in_proj-output gradient)
  const KView vdx = with_layout<UL>(p.dx, p.x), vddt = with_layout<UL>(p.ddt, p.x);
  const KView vB = p.Bm, vC = with_layout<UL>(p.Cm, p.Bm);
  const bool xt = vx.s1 == 1, dtt = vdt.s1 == 1, bt = vB.s1 == 1, ctt = vC.s1 == 1;
  const bool gt = vg.s1 == 1, dxt = vdx.s1 == 1, ddtt = vddt.s1 == 1;
  const CT *ypre = (const CT *)p.ypre;
  CT biasv[WaveTile<IT, CT, CK, CW, UL>::E], dskv[WaveTile<IT, CT, CK, CW, UL>::E];
  tile_bias<CT, CK, CW>(biasv, p.has_bias, p.bias, dw, D, dtt, lane);
  tile_bias<CT, CK, CW>(dskv, p.has_D, p.Dsk, dw, D, dxt, lane);  // D skip in the dx store mapping

  // Global reads run two chunks ahead (chunks are walked from the last to the first): tiles
  // ping-pong between two register sets, each refilled as soon as its chunk is staged in LDS.
  // Every load is unconditional (clamped addresses), so waiting for one chunk's tiles leaves
  // the prefetches and earlier stores in flight.  A chunk k < 0 is inert (all inputs zero, no
  // stores): chunks always run in pairs, and the loop is entered with the same memory traffic
  // in flight as on its back edge.  In an inert chunk the adjoint first takes the step to
  // a_0 dh_0 and then stays, which is what the dh0 epilogue expects.
  constexpr int E1 = WaveTile<IT, CT, CK, CW, UL>::E;
  // dD and d_bias: each lane accumulates over the chunks the terms of the (step slot, channel)
  // elements it stores (a fixed mapping), and the channel totals add the CK slots at the end.
  CT dDp[E1], dbp[E1];
#pragma unroll
  for (int i = 0; i < E1; ++i) dDp[i] = dbp[i] = 0;
  struct Tiles {
    WaveTile<IT, CT, CK, CW, UL> x, dt, g, z;
    WaveTile<IT, CT, CK, NP, UL> B, C;
    LowRankTile<IT, CT, CK> lr;
    CT yp[E1];
    CT ck;
  };
  const KView vzl = p.has_z ? vz : vx;
  const int dc = dval ? d : 0;
  // With a uniform layout x, delta, dout, z share one set of lane offsets (B, C another), and
  // they and the saved pre-gate output are read through raw buffers over one batch row.
  constexpr int ES = (int)sizeof(IT), EB = WaveTile<IT, CT, CK, NP, UL>::E;
  uint32_t offX[E1], offB[EB], offY[E1], offZ[E1];
  tile_offsets<CK, CW>(offX, vx, dw, xt, lane, ES);
  tile_offsets<CK, CW>(offZ, vzl, dw, gt, lane, ES);  // the gate (e.g. the in_proj split) may differ
  tile_offsets<CK, NP>(offB, vB, 0, bt, lane, ES);
  const KView vy{ypre, xt ? 1 : (int64_t)D, xt ? 1 : (int64_t)D, xt ? (int64_t)L : 1};  // ypre's (t, d) strides
  tile_offsets<CK, CW>(offY, vy, dw, gt, lane, (int)sizeof(CT));
  const __amdgpu_buffer_rsrc_t empty = __builtin_amdgcn_make_buffer_rsrc((void *)p.x.p, (short)0, 0, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rbx = row_buffer(vx, b, L, D, ES);
  const __amdgpu_buffer_rsrc_t rbdt = LR ? empty : row_buffer(vdt, b, L, D, ES);
  // low-rank delta: input block reads and the weight rows in LDS
  __amdgpu_buffer_rsrc_t rblr = empty;
  uint32_t offLR = 0, tstepLR = 0;
  bool rvLR = false;
  if constexpr (LR) {
    rblr = row_buffer(p.dtl, b, L, p.lowrank, ES);
    lowrank_offsets(p.dtl, p.lowrank, lane, ES, offLR, tstepLR, rvLR);
    lowrank_weights<CT, CW>(S.wr, p.dtw, p.lowrank, dw, D, lane);
  }
  const __amdgpu_buffer_rsrc_t rbg = row_buffer(vg, b, L, D, ES), rbz = row_buffer(vzl, b, L, D, ES);
  const __amdgpu_buffer_rsrc_t rbB = row_buffer(vB, b, L, N, ES), rbC = row_buffer(vC, b, L, N, ES);
  const __amdgpu_buffer_rsrc_t rby = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(ypre ? ypre + b * p.L * p.D : (const CT *)p.ckpt), (short)0, (int)(ypre ? p.L * p.D * sizeof(CT) : 0),
      kBufferFlags);
  auto load = [&](Tiles &T, int k) {
    const int kc = k < 0 ? 0 : k;
    const int t0 = kc * CK;
    if constexpr (LR) T.lr.load(rblr, offLR + (uint32_t)(t0 * (int)p.dtl.s1 * ES), tstepLR, rvLR);
    if constexpr (UL) {
      const uint32_t tx_ = (uint32_t)(t0 * (int)vx.s1 * ES), tb_ = (uint32_t)(t0 * (int)vB.s1 * ES);
      T.x.load_buf(rbx, offX, tx_);
      T.dt.load_buf(rbdt, offX, tx_);
      T.g.load_buf(rbg, offX, tx_);
      T.z.load_buf(rbz, offZ, (uint32_t)(t0 * (int)vzl.s1 * ES));
      T.B.load_buf(rbB, offB, tb_);
      T.C.load_buf(rbC, offB, tb_);
      if (p.has_z) {
        const uint32_t ty_ = (uint32_t)(t0 * (int)vy.s1 * (int)sizeof(CT));
#pragma unroll
        for (int i = 0; i < E1; ++i) T.yp[i] = buf_load<CT>(rby, offY[i] + ty_);
      }
    } else {
      T.x.load(vx, b, t0, L, dw, D, xt, lane);
      T.dt.load(vdt, b, t0, L, dw, D, dtt, lane);
      T.g.load(vg, b, t0, L, dw, D, gt, lane);
      T.z.load(vzl, b, t0, L, dw, D, gt, lane);
      T.B.load(vB, b, t0, L, 0, N, bt, lane);
      T.C.load(vC, b, t0, L, 0, N, ctt, lane);
      if (p.has_z) {
#pragma unroll
        for (int i = 0; i < E1; ++i) {
          int t, cc;
          tc_of<CK, CW>(lane + i * kWave, gt, t, cc);
          T.yp[i] = ypre[ypre_index(!xt, b, min(t0 + t, L - 1), min(dw + cc, D - 1), p.L, p.D)];
        }
      }
    }
    T.ck = ((const CT *)p.ckpt)[((b * p.nchunks + (kc > 0 ? kc - 1 : 0)) * p.D + dc) * NP + n];
  };

  auto chunk = [&](Tiles &T, int k) {
    const bool live = k >= 0;
    const int t0 = live ? k * CK : 0;
    const int Lc = live ? L : 0;  // time bound of this chunk's elements (0: inert)
    const int buf = k & 1;
    // ---------------------------------------------------------------- stage
    {
      T.x.store(S.x, xt, lane, t0, Lc, dw, D);
      if constexpr (LR) {
        T.lr.store(S.lr, lane);
        wave_lds_sync();
        lowrank_delta<IT, CT, CK, CW, UL>(T.dt, S.lr, S.wr, dtt, lane);
      }
      store_delta_w<IT, CT, CK, CW, WL::CKP, UL>(T.dt, S.dt, S.sg, dtt, lane, p.softplus, biasv, dw, D, t0, Lc);
      T.B.store(S.B, bt, lane, t0, Lc, 0, N);
      T.C.store(S.C, ctt, lane, t0, Lc, 0, N);
      // dy = dout * silu(z); dz = dout * (y + D x) * silu'(z), from the saved pre-gate output
#pragma unroll
      for (int i = 0; i < E1; ++i) {
        const int e = lane + i * kWave;
        if (e >= CK * CW) break;
        int t, cc;
        tc_of<CK, CW>(e, gt, t, cc);
        const int tg = t0 + t, dd = dw + cc;
        CT g = 0;
        if (tg < Lc && dd < D) {
          g = T.g.v[i];
          if (p.has_z) {
            const CT zv = T.z.v[i];
            const CT sgz = sigmoid_ct<CT>(zv);
            Conv<IT>::store(vpw<IT>(vdz) + b * vdz.s0 + row_off<UL>(tg, dd, vdz.s1, vdz.s2),
                            g * T.yp[i] * sgz * ((CT)1 + zv * ((CT)1 - sgz)));
            g = g * zv * sgz;
          }
        }
        S.dy[cc][t] = g;
      }
    }
    CT hh[CK + 1], aa[CK], cc_[CK], bxs[CK];  // bxs: B x of each step, kept for the reverse walk
    hh[0] = k <= 0 ? h0v : T.ck;
    wave_lds_sync();
    load(T, k - 2);

    // ---------------------------------------------------------------- recompute states
    {
      CT rdt[RB], rx[RB], rB[RB];
      lds_row(&S.dt[c][0], rdt);
      lds_row(&S.x[c][0], rx);
      lds_row(&S.B[n][0], rB);
#pragma unroll
      for (int q = 0; q < CK / RB; ++q) {
        CT bx[RB];
#pragma unroll
        for (int tt = 0; tt < RB; ++tt) {
          const int t = q * RB + tt;
          if constexpr (M1) disc_zoh_m1(rdt[tt], ac, aa[t], cc_[t]);
          else disc<METHOD>(rdt[tt], ac, aa[t], cc_[t]);
          bxs[t] = rB[tt] * rx[tt];
          bx[tt] = bcoef<METHOD>(rdt[tt], cc_[t]) * bxs[t];
        }
        if (q + 1 < CK / RB) {
          lds_row(&S.dt[c][(q + 1) * RB], rdt);
          lds_row(&S.x[c][(q + 1) * RB], rx);
          lds_row(&S.B[n][(q + 1) * RB], rB);
        }
#pragma unroll
        for (int tt = 0; tt < RB; ++tt) {
          const int t = q * RB + tt;
          if constexpr (M1) hh[t + 1] = fma(aa[t], hh[t], hh[t] + bx[tt]);
          else hh[t + 1] = fma(aa[t], hh[t], bx[tt]);
        }
      }
    }

    // ---------------------------------------------------------------- reverse walk
#pragma unroll
    for (int half = CK / RH - 1; half >= 0; --half) {
      CT rdt[RB], rx[RB], rdy[RB], rB[RB], rC[RB];
#pragma unroll
      for (int q = RH / RB - 1; q >= 0; --q) {
        const int tb = half * RH + q * RB;  // first step of the batch
        lds_row(&S.dt[c][tb], rdt);
        lds_row(&S.x[c][tb], rx);
        lds_row(&S.dy[c][tb], rdy);
        lds_row(&S.B[n][tb], rB);
        lds_row(&S.C[n][tb], rC);
#pragma unroll
        for (int tt = RB - 1; tt >= 0; --tt) {
          const int t = tb + tt;
          const int slot = t - half * RH;
          const CT dtv = rdt[tt], xv = rx[tt], dyv = rdy[tt], Bv = rB[tt], Cv = rC[tt];
          if constexpr (M1) dh64 = fma(dh64, (double)a_next, dh64 + (double)(dyv * Cv));
          else dh64 = fma(dh64, (double)a_next, (double)(dyv * Cv));
          const CT lam = (CT)dh64;
          a_next = aa[t];
          const CT hp = hh[t], Bx = bxs[t];
          const CT pC = dyv * hh[t + 1];
          const CT dhc = lam * bcoef<METHOD>(dtv, cc_[t]);
          const CT px = dhc * Bv;
          const CT pB = dhc * xv;
          // ddelta_t per state = lambda (da/dz A h_{t-1} + db/ddelta / (B x) B x)
          CT pD;
          if constexpr (METHOD == 0) {  // da/dz = db/ddelta-factor = a; a (A h_{t-1} + B x) = A h_t + B x
            pD = lam * fma(ac.A, hh[t + 1], Bx);
          } else if constexpr (METHOD == 1) {  // da/dz = a, db/ddelta-factor = 1
            pD = fma(lam * aa[t] * ac.A, hp, lam * Bx);
          } else {  // both factors u^2 with u = 1 / (1 - z/2), held in cc_
            pD = lam * (cc_[t] * cc_[t]) * fma(ac.A, hp, Bx);
          }
          dA_acc = fma(dtv, pD, fma(-dhc, Bx, dA_acc));
          S.pn[slot][c][0][n] = px;
          S.pn[slot][c][1][n] = pD;
          S.pd[slot][c][n][0] = pB;
          S.pd[slot][c][n][1] = pC;
        }
      }
      wave_lds_sync();
      // Every partial this lane adds is read before the first sum is written: a write between
      // them would order the later reads after it, one LDS round trip per sum.
      constexpr int NPN = (RH * CW * 2 + kWave - 1) / kWave, NPD = (RH * NP + kWave - 1) / kWave;
      CT part[NPN][NP], pdv[NPD][CW][2];
#pragma unroll
      for (int i = 0; i < NPN; ++i) {
        const int e = lane + i * kWave;
        if (e >= RH * CW * 2) break;
        const int q = e % 2, cn = (e / 2) % CW, tt = e / (2 * CW);
        lds_row(&S.pn[tt][cn][q][0], part[i]);
      }
#pragma unroll
      for (int i = 0; i < NPD; ++i) {
        const int e = lane + i * kWave;
        if (e >= RH * NP) break;
        const int tt = e / NP, nn = e % NP;
#pragma unroll
        for (int j = 0; j < CW; ++j) {
          pdv[i][j][0] = S.pd[tt][j][nn][0];
          pdv[i][j][1] = S.pd[tt][j][nn][1];
        }
      }
      // (dx, ddelta): sum over the NP states of a channel, one (step, channel, quantity) per lane
#pragma unroll
      for (int i = 0; i < NPN; ++i) {
        const int e = lane + i * kWave;
        if (e >= RH * CW * 2) break;
        const int q = e % 2, cn = (e / 2) % CW, tt = e / (2 * CW);
        CT sum = 0;
#pragma unroll
        for (int j = 0; j < NP; ++j) sum += part[i][j];
        (q == 0 ? S.gx : S.gd)[cn][half * RH + tt] = sum;
      }
      // (dB, dC): sum over the wavefront's CW channels
#pragma unroll
      for (int i = 0; i < NPD; ++i) {
        const int e = lane + i * kWave;
        if (e >= RH * NP) break;
        const int tt = e / NP, nn = e % NP;
        CT sb = 0, sc = 0;
#pragma unroll
        for (int j = 0; j < CW; ++j) {
          sb += pdv[i][j][0];
          sc += pdv[i][j][1];
        }
        const int t = half * RH + tt;
        if constexpr (WPB > 1) {
          sh.dbc[buf][wv][t][nn][0] = sb;
          sh.dbc[buf][wv][t][nn][1] = sc;
        } else {
          if (t0 + t < Lc) {
            const int64_t off = ((b * p.ntiles + tile) * p.L + t0 + t) * NP + nn;
            ((CT *)p.ws_dB)[off] = sb;
            ((CT *)p.ws_dC)[off] = sc;
          }
        }
      }
      wave_lds_sync();
    }

    // ---------------------------------------------------------------- store
#pragma unroll
    for (int i = 0; i < (CK * CW + kWave - 1) / kWave; ++i) {
      const int e = lane + i * kWave;
      if (e >= CK * CW) break;
      int t, cc;
      tc_of<CK, CW>(e, dxt, t, cc);
      const int tg = t0 + t, dd = dw + cc;
      if (tg >= Lc || dd >= D) continue;
      CT gx = S.gx[cc][t];
      const CT dyv = S.dy[cc][t];  // read with gx: one LDS round trip
      if (p.has_D) gx += dyv * dskv[i];
      Conv<IT>::store(vpw<IT>(vdx) + b * vdx.s0 + row_off<UL>(tg, dd, vdx.s1, vdx.s2), gx);
    }
#pragma unroll
    for (int i = 0; i < (CK * CW + kWave - 1) / kWave; ++i) {
      const int e = lane + i * kWave;
      if (e >= CK * CW) break;
      int t, cc;
      tc_of<CK, CW>(e, ddtt, t, cc);
      const int tg = t0 + t, dd = dw + cc;
      if (tg >= Lc || dd >= D) continue;
      const CT gd = S.gd[cc][t], sg = S.sg[cc][t];
      dbp[i] = fma(gd, sg, dbp[i]);
      dDp[i] = fma(S.dy[cc][t], S.x[cc][t], dDp[i]);
      Conv<IT>::store(vpw<IT>(vddt) + b * vddt.s0 + row_off<UL>(tg, dd, vddt.s1, vddt.s2), gd * sg);
    }
    if constexpr (WPB > 1) {
      lds_barrier();  // every wavefront's (dB, dC) sums of this chunk are in sh.dbc[buf]
      for (int e = tid; e < CK * NP * 2; e += NT) {
        const int q = e % 2, nn = (e / 2) % NP, t = e / (2 * NP);
        if (t0 + t >= Lc) continue;
        CT v = 0;
#pragma unroll
        for (int w = 0; w < WPB; ++w) v += sh.dbc[buf][w][t][nn][q];
        const int64_t off = ((b * p.ntiles + tile) * p.L + t0 + t) * NP + nn;
        ((CT *)(q == 0 ? p.ws_dB : p.ws_dC))[off] = v;
      }
    }
    wave_lds_sync();
    };

  Tiles T0, T1;
  const int K = p.nchunks;
  load(T0, K - 1);
  load(T1, K - 2);
  chunk(T0, K - 1);
  chunk(T1, K - 2);
  for (int k = K - 3; k >= 0; k -= 2) {
    chunk(T0, k);
    chunk(T1, k - 1);
  }

  if (dval) ((double *)p.ws_dA)[(b * p.D + d) * NP + n] = (double)(dA_acc * ac.invA);
  if (p.has_dh0 && dval && nval)
    vstore<CT>(p.dh0, b * p.dh0.s0 + d * p.dh0.s1 + n * p.dh0.s2,
               (CT)(M1 ? fma(dh64, (double)a_next, dh64) : dh64 * (double)a_next));
#pragma unroll
  for (int i = 0; i < E1; ++i) {
    const int e = lane + i * kWave;
    if (e >= CK * CW) break;
    int t, cc;
    tc_of<CK, CW>(e, ddtt, t, cc);
    S.gx[cc][t] = dDp[i];
    S.gd[cc][t] = dbp[i];
  }
  wave_lds_sync();
  if (lane < CW && dw + lane < D) {
    CT sD = 0, sb = 0;
#pragma unroll
    for (int t = 0; t < CK; ++t) {
      sD += S.gx[lane][t];
      sb += S.gd[lane][t];
    }
    ((CT *)p.ws_dD)[b * p.D + dw + lane] = sD;
    ((CT *)p.ws_db)[b * p.D + dw + lane] = sb;
  }
}

// Fixed-order final reductions: dB/dC over channel tiles, dA/dD/d_bias over the batch.
// Each sum runs over its terms in index order; the reads of a group of kFinGroup terms are
// issued together ahead of their adds (the sums are latency-bound chains of dependent
// round trips otherwise).  With V4 a lane sums four consecutive states of dB or of dC with
// 16-byte reads (float partials, 16-byte aligned, np a multiple of 4).
constexpr int kFinGroup = 4;

template <typename CT>
__device__ inline CT fin_sum(const CT *src, int64_t stride, int64_t count) {
  return ordered_sum<kFinGroup>(src, stride, count);
}

__device__ inline float4 fin_sum4(const float4 *src, int64_t stride, int count) {
  float4 s = {0.f, 0.f, 0.f, 0.f};
  int k = 0;
  for (; k + kFinGroup <= count; k += kFinGroup) {
    float4 v[kFinGroup];
#pragma unroll
    for (int u = 0; u < kFinGroup; ++u) v[u] = src[(k + u) * stride];
#pragma unroll
    for (int u = 0; u < kFinGroup; ++u) {
      s.x += v[u].x; s.y += v[u].y; s.z += v[u].z; s.w += v[u].w;
    }
  }
  for (; k < count; ++k) {
    const float4 v = src[k * stride];
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  return s;
}

// Lanes handling dB / dC with V4 (two quantities, np / 4 lanes per (b, t)) or without.
__host__ __device__ inline int64_t fin_bc_lanes(const FinParams &p, bool v4) {
  return v4 ? 2 * p.B * p.L * (p.np / 4) : p.B * p.L * p.N;
}

template <typename OT, typename CT, bool V4>
__global__ void __launch_bounds__(256) k_bwd_finalize(const FinParams p) {
  const int64_t nBC = fin_bc_lanes(p, V4);
  const int64_t nDN = p.D * p.N;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nBC) {
    const int64_t tstride = p.L * p.np;  // between the partials of consecutive tiles
    if constexpr (V4) {
      const int q4 = p.np / 4;
      const int64_t half = nBC / 2;
      const bool isC = i >= half;
      const int64_t r = isC ? i - half : i;
      const int64_t n4 = r % q4, t = (r / q4) % p.L, b = r / (q4 * p.L);
      const float4 *src = (const float4 *)(isC ? p.ws_dC : p.ws_dB) + (b * p.ntiles * p.L + t) * q4 + n4;
      const float4 s = fin_sum4(src, tstride / 4, p.ntiles);
      const KView &o = isC ? p.dC : p.dB;
      const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t nn = n4 * 4 + k;
        if (nn < p.N) Conv<OT>::store(vpw<OT>(o) + b * o.s0 + t * o.s1 + nn * o.s2, sv[k]);
      }
    } else {
      const int64_t nn = i % p.N, t = (i / p.N) % p.L, b = i / (p.N * p.L);
      const int64_t off0 = (b * p.ntiles * p.L + t) * p.np + nn;
      const CT sb = fin_sum((const CT *)p.ws_dB + off0, tstride, p.ntiles);
      const CT sc = fin_sum((const CT *)p.ws_dC + off0, tstride, p.ntiles);
      Conv<OT>::store(vpw<OT>(p.dB) + b * p.dB.s0 + t * p.dB.s1 + nn * p.dB.s2, sb);
      Conv<OT>::store(vpw<OT>(p.dC) + b * p.dC.s0 + t * p.dC.s1 + nn * p.dC.s2, sc);
    }
    return;
  }
  const int64_t j = i - nBC;
  if (j < nDN) {
    const int64_t d = j / p.N, nn = j % p.N;
    // the row partials are float64 (each sums a row's or segment's steps): their sum, then one
    // rounding to the output type
    double s = fin_sum((const double *)p.ws_dA + d * p.np + nn, p.D * p.np, p.rows);
    if (p.a_log) s *= -exp((double)vload<CT>(p.A, d * p.A.s0 + nn * p.A.s1));  // dA_log = dA * A
    vstore<CT>(p.dA, d * p.dA.s0 + nn * p.dA.s1, (CT)s);
    return;
  }
  const int64_t k = j - nDN;
  if (k < p.D) {
    if (p.has_D) vstore<CT>(p.dD, k * p.dD.s0, fin_sum((const CT *)p.ws_dD + k, p.D, p.rows));
    if (p.has_bias) vstore<CT>(p.dbias, k * p.dbias.s0, fin_sum((const CT *)p.ws_db + k, p.D, p.rows));
  }
}

// ------------------------------------------------------------------ float kernels (row tiles)
// The float-compute backward (float32 / bf16 / fp16 inputs, float32 state), NP >= 16.  Same
// per-chunk structure as k_bwd, with the changes of the forward's row-tile kernel:
//   * x, delta (bias / softplus applied), dy = dout silu(z) and the softplus derivative stay in
//     one register per lane (row tiles) and reach each step's lanes by DPP row broadcast; B is
//     read from LDS once per chunk and kept in registers from the recompute to the walk back;
//   * the sums over the states of the dx / ddelta terms land directly in the row-tile lanes
//     that store them (no LDS round trip for the stores);
//   * the adjoint keeps float64 accuracy with one float64 add per step: the step's increment
//     (a - 1) lambda + dy C is formed in float32 (it is small against lambda, and dy C carries
//     its own float32 rounding in any case) and accumulated into a float64 lambda;
//   * buffer addresses take the chunk offset as a scalar operand.
// Time segments (few batch rows x channels, long L): each segment walks its own chunks from the
// adjoint carried into it.  A summary pass (SUM) gives each segment's zero-start adjoint at its
// first step times that step's decay (E) and the product of its decays (P); k_bwd_carry turns
// them into the adjoint entering every segment, the reverse of the forward's segment carry.
// (dx, ddelta) terms of half a chunk at [c * PCS + (t * 2 + q) * NPP + n]: a channel block is
// padded by 16 floats, so the two channels of a half-wavefront write 32 distinct banks.  (Reads
// of the rows in the forward's conflict-free order, with the reducers remapped to match, took
// 4 extra cycles fewer per 16-byte read and no less time: this kernel is not bound by LDS.)
template <int NP, bool LR>
struct BwdwLds {
  static constexpr int CW = kWave / NP, CKP = ck_pad(4), NPP = np_pad(4, NP), RH = 8, PCS = 2 * RH * NPP + 16;
  float B[NP][CKP];
  float C[NP][CKP];
  float pn[CW * PCS];
  float lr[LR ? kCK : 1][lr_pad(4)];
  float wr[LR ? CW : 1][lr_pad(4)];
};

template <typename IT, int NP, int METHOD, bool UL, bool SUM, bool LR>
__global__ void __launch_bounds__(kWave * bwdw_waves(NP)) k_bwdw(const BwdParams p) {
  typedef BwdwLds<NP, LR> WL;
  typedef RowGeo<NP> G;
  typedef RowTile<IT, NP, UL> RT;
  constexpr int CW = G::CW, CK = kCK, RH = WL::RH, WPB = bwdw_waves(NP), NT = WPB * kWave;
  constexpr bool M1 = METHOD == 0;
  // (dB, dC) of half a chunk for every channel of the workgroup, by half: rows of CH channels
  // padded to CHP (rows 16-byte aligned for the reducers' reads).  The state lanes
  // write their factors -- dB_t[n] = sum_c (lambda cf)_t[c][n] x_t[c] and dC_t[n] = sum_c
  // h_t[c][n] dy_t[c] -- and after a barrier TPI threads form each (step, quantity, state)
  // row's dot product with the step's x or dy row (staged per chunk, by chunk parity), IPT
  // rows per thread: one FMA per term where a product per state lane and an add were two.
  constexpr int CH = WPB * CW, CHP = CH + 4, NITEM = RH * 2 * NP;
  constexpr int TPI = NT >= NITEM ? NT / NITEM : 1, IPT = NITEM > NT ? NITEM / NT : 1, CPT = CH / TPI;
  static_assert(TPI <= 2 && CPT % 4 == 0 && NITEM == IPT * (NT / TPI), "reduction layout");
  __shared__ __align__(16) WL lds_all[WPB];
  __shared__ __align__(16) float pdw[2][RH][2][NP][CHP];
  __shared__ __align__(16) float xdy[2][2][kCK][CHP];  // [chunk parity][x, dy][step][channel]

  const int tid = threadIdx.x;
  const int lane = tid % kWave, wv = tid / kWave;
  WL &S = lds_all[wv];
  const int c = lane / NP, n = lane % NP;
  const int tj = G::step(lane), tc = G::chan(lane);
  const int64_t b = blockIdx.y / p.nseg;
  const int seg = (int)(blockIdx.y % p.nseg);
  if (SUM && seg == 0) return;  // the first segment's summary is never used
  const int k0 = seg * p.seg_chunks;
  const int k1 = k0 + p.seg_chunks < p.nchunks ? k0 + p.seg_chunks : p.nchunks;
  const int tile = xcd_tile();
  const int dw = (tile * WPB + wv) * CW;
  const int d = dw + c;
  const bool dval = d < p.D, nval = n < p.N;
  const bool tval = dw + tc < p.D;
  const int L = (int)p.L, D = (int)p.D, N = (int)p.N;
  const int64_t sidx = ((b * p.nseg + seg) * p.D + d) * NP + n;  // (B, nseg, D, NP)

  float Av = -1.0f;
  if (dval && nval) {
    Av = vload<float>(p.A, d * p.A.s0 + n * p.A.s1);
    if (p.a_log) Av = -__expf(Av);  // models/mamba.py:81
  }
  const AConst<float> ac = make_aconst(Av);
  // the adjoint entering the segment's last step: dlast, or the carry of the later segments
  double lam = 0.0;
  if (!SUM && dval && nval) {
    if (p.nseg > 1) lam = ((const double *)p.seg_mu)[sidx];
    else if (p.has_dlast) lam = (double)vload<float>(p.dlast, b * p.dlast.s0 + d * p.dlast.s1 + n * p.dlast.s2);
  }
  float lamf = (float)lam;
  float m_next = M1 ? 0.0f : 1.0f;  // a - 1 (ZOH) or a of the step after the current one
  float prod = 1.0f;                // summary: product of the segment's decays
  // summary, ZOH and Euler: that product is exp(A sum_t delta_t), from the lanes' row-tile
  // deltas added once per chunk (float64) and summed over the row at the end
  constexpr bool PSUM = SUM && METHOD != 2;
  double dsum = 0.0;
  float h0v = 0.0f;
  if (!SUM && p.has_h0 && dval && nval) h0v = vload<float>(p.h0, b * p.h0.s0 + d * p.h0.s1 + n * p.h0.s2);
  // dA sums every step of the sequence: each chunk's 16 terms in float32, the chunk sums in
  // float64 (a float32 running sum over a long sequence loses the small elements of dA)
  // dD and d_bias: one term per chunk and lane, summed over the sequence in float64
  double dA64 = 0.0, dDp = 0.0, dbp = 0.0;
  const float biasv = p.has_bias && tval ? vload<float>(p.bias, (int64_t)(dw + tc) * p.bias.s0) : 0.0f;
  const float dskv = p.has_D && tval ? vload<float>(p.Dsk, (int64_t)(dw + tc) * p.Dsk.s0) : 0.0f;

  const KView vx = p.x, vdt = with_layout<UL>(p.dt, p.x), vz = p.z;
  const KView vg = with_layout<UL>(p.dout, p.x), vdz = p.dz;
  const KView vdx = with_layout<UL>(p.dx, p.x), vddt = with_layout<UL>(p.ddt, p.x);
  const KView vB = p.Bm, vC = with_layout<UL>(p.Cm, p.Bm);
  const bool bt = vB.s1 == 1, ctt = vC.s1 == 1;
  const KView vzl = p.has_z ? vz : vx;
  const float *ypre = (const float *)p.ypre;
  struct Tiles {
    RT x, dt, g, z, yp;
    WaveTile<IT, float, CK, NP, UL> B, C;
    LowRankTile<IT, float, CK> lr;
    float ck;
  };
  constexpr int ES = (int)sizeof(IT), EB = WaveTile<IT, float, CK, NP, UL>::E;
  const uint32_t offX = RT::offset(vx, dw, lane), offZ = RT::offset(vzl, dw, lane);
  const uint32_t offDZ = p.has_z ? RT::offset(vdz, dw, lane) : 0u;
  uint32_t offB[EB];
  tile_offsets<CK, NP>(offB, vB, 0, bt, lane, ES);
  const __amdgpu_buffer_rsrc_t empty = flat_buffer(p.x.p, 0);
  const RowRef rx = row_ref(vx, b, L, D, ES), rdt = row_ref(LR ? vx : vdt, b, L, D, ES);
  const RowRef rg = row_ref(vg, b, L, D, ES), rz = row_ref(vzl, b, L, D, ES);
  const RowRef rB = row_ref(vB, b, L, N, ES), rC = row_ref(vC, b, L, N, ES);
  const RowRef rdx = row_ref(vdx, b, L, D, ES), rddt = row_ref(vddt, b, L, D, ES);
  const RowRef rdz = row_ref(p.has_z ? vdz : vdx, b, L, D, ES);
  const int64_t ckrow = (int64_t)p.nchunks * p.D * NP;
  const RowRef rk = flat_ref((const float *)p.ckpt + b * ckrow, ckrow * 4);
  const RowRef ry = flat_ref(ypre ? ypre + b * p.L * p.D : p.x.p, ypre ? p.L * p.D * 4 : 0);
  // the (b, tile) rows of the dB / dC partials, (L, NP) each (the host keeps them below 2^31 bytes)
  const int64_t wrow = (b * p.ntiles + tile) * p.L * NP;
  const RowRef rwB = flat_ref((const float *)p.ws_dB + wrow, p.L * NP * 4);
  const RowRef rwC = flat_ref((const float *)p.ws_dC + wrow, p.L * NP * 4);
  const uint32_t offK = (uint32_t)((dval ? d : 0) * NP + n) * 4u;
  // the float forward saves the pre-gate output as (B, D, L)
  const uint32_t offY = (uint32_t)(ypre_index(false, 0, tj, dw + tc, p.L, p.D) * 4);
  const uint32_t tstepY = (uint32_t)(CK * 4);
  __amdgpu_buffer_rsrc_t rblr = empty;
  uint32_t offLR = 0, tstepLR = 0;
  bool rvLR = false;
  if constexpr (LR) {
    rblr = row_buffer(p.dtl, b, L, p.lowrank, ES);
    lowrank_offsets(p.dtl, p.lowrank, lane, ES, offLR, tstepLR, rvLR);
    lowrank_weights<float, CW>(S.wr, p.dtw, p.lowrank, dw, D, lane);
  }

  // Loads run one chunk ahead of the walk (chunks go from the last to the first): a chunk's
  // tiles are requested as soon as the previous chunk is staged.  Every load is unconditional,
  // and a chunk k < k0 re-reads chunk k0 and is inert.
  auto load = [&](Tiles &T, int k) {
    const int kc = k < k0 ? k0 : k;
    const int t0 = kc * CK;
    if constexpr (LR) T.lr.load(rblr, offLR + (uint32_t)(t0 * (int)p.dtl.s1 * ES), tstepLR, rvLR);
    if constexpr (UL) {
      // the chunk offset goes into the range-checked vector offset: the ragged last chunk's
      // lanes past the row read 0 (a scalar offset would escape the check)
      const uint32_t ox = offX + (uint32_t)(t0 * (int)vx.s1 * ES), tb_ = (uint32_t)(t0 * (int)vB.s1 * ES);
      if constexpr (!SUM) T.x.v = buf_load<IT>(rx.rsrc(), ox);
      if constexpr (!LR) T.dt.v = buf_load<IT>(rdt.rsrc(), ox);
      T.g.v = buf_load<IT>(rg.rsrc(), ox);
      T.z.v = buf_load<IT>(rz.rsrc(), offZ + (uint32_t)(t0 * (int)vzl.s1 * ES));
      if constexpr (!SUM) {
#pragma unroll
        for (int i = 0; i < EB; ++i) T.B.v[i] = buf_load<IT>(rB.rsrc(), offB[i] + tb_);
      }
#pragma unroll
      for (int i = 0; i < EB; ++i) T.C.v[i] = buf_load<IT>(rC.rsrc(), offB[i] + tb_);
      if constexpr (!SUM) {
        T.yp.v = buf_load<float>(ry.rsrc(), offY + (uint32_t)kc * tstepY);
        T.ck = buf_load_s<float>(rk.rsrc(), offK, (uint32_t)((kc > 0 ? kc - 1 : 0) * (int)p.D * NP * 4));
      }
    } else {
      if constexpr (!SUM) T.x.load(vx, b, t0, L, dw, D, lane);
      if constexpr (!LR) T.dt.load(vdt, b, t0, L, dw, D, lane);
      T.g.load(vg, b, t0, L, dw, D, lane);
      T.z.load(vzl, b, t0, L, dw, D, lane);
      if constexpr (!SUM) T.B.load(vB, b, t0, L, 0, N, bt, lane);
      T.C.load(vC, b, t0, L, 0, N, ctt, lane);
      if constexpr (!SUM) {
        T.yp.v = ypre ? ypre[ypre_index(false, b, min(t0 + tj, L - 1), min(dw + tc, D - 1), p.L, p.D)] : 0.0f;
        T.ck = ((const float *)p.ckpt)[((b * p.nchunks + (kc > 0 ? kc - 1 : 0)) * p.D + (dval ? d : 0)) * NP + n];
      }
    }
  };

  float Rh[2];  // the half chunks' state sums: lane (r, j) holds step 8 h + j % 8, quantity j / 8
  // The (dB, dC) sums over the workgroup's channels are software-pipelined: a half chunk's LDS
  // reads are issued right after its barrier, and summed and stored after the next half's walk,
  // whose work hides their latency (the two wavefronts of a SIMD belong to one workgroup and
  // reach the barrier together, so nothing else would).  dq_t: first step of the pending half;
  // dq_L: the sequence length, 0 when nothing is pending (every store masked).
  float dq[IPT][CPT], dqw[IPT][CPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i)
#pragma unroll
    for (int j = 0; j < CPT; ++j) dq[i][j] = dqw[i][j] = 0.0f;
  int dq_t = 0, dq_L = 0;
  // Reducer thread -> (row item, part of its channels).  With two threads per item the 16 lanes
  // of a 16-byte read phase take 16 consecutive items of one part (16 distinct rows, distinct
  // banks); a thread's partner is the lane 16 apart in its 32-lane half.
  auto red_item = [&](int i, int &item, int &part) {
    if constexpr (TPI == 2) {
      part = (tid >> 4) & 1;
      item = (tid >> 5) * 16 + (tid & 15) + i * (NT / TPI);
    } else {
      part = 0;
      item = tid + i * NT;
    }
  };
  auto dq_flush = [&]() {
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      int item, part;
      red_item(i, item, part);
      const int st = item / (2 * NP), q = (item / NP) % 2, nn = item % NP;
      float sum = dot_sum(dq[i], dqw[i]);
      if constexpr (TPI == 2)  // the partner's channels (lane ^ 16; the same bits in both lanes)
        sum += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, sum), 0x401F));
      const int tg = dq_t + st;
      if constexpr (UL) {  // two masked stores: q differs between the lanes of a wavefront
        const uint32_t ow = (uint32_t)((st * NP + nn) * 4), tw = (uint32_t)(dq_t * NP * 4);
        const bool ok = part == 0 && tg < dq_L;
        buf_store_s<float>(rwB.rsrc(), ow, tw, ok && q == 0, sum);
        buf_store_s<float>(rwC.rsrc(), ow, tw, ok && q == 1, sum);
      } else if (part == 0 && tg < dq_L) {
        ((float *)(q == 0 ? p.ws_dB : p.ws_dC))[((b * p.ntiles + tile) * p.L + tg) * NP + nn] = sum;
      }
    }
  };
  auto chunk = [&](Tiles &T, int k) {
    const bool live = k >= k0;
    const int t0 = (live ? k : k0) * CK;
    const int Lc = live ? L : 0;
    const bool ev = t0 + tj < Lc && tval;
    const int par = k & 1;
    // ------------------------------------------------------------ stage
    if constexpr (!SUM) T.B.store(S.B, bt, lane, t0, Lc, 0, N);
    T.C.store(S.C, ctt, lane, t0, Lc, 0, N);
    const float xv = ev ? T.x.v : 0.0f;
    float dv;
    if constexpr (LR) {
      T.lr.store(S.lr, lane);
      wave_lds_sync();
      float a_[kLR], w_[kLR];
      lds_row(&S.lr[tj][0], a_);
      lds_row(&S.wr[tc][0], w_);
      dv = 0.0f;
#pragma unroll
      for (int r = 0; r < kLR; ++r) dv = fmaf(a_[r], w_[r], dv);
    } else {
      dv = T.dt.v;
    }
    dv += biasv;
    float sgv = 1.0f;
    if (p.softplus) {
      sgv = sigmoidf(dv);
      dv = softplusf(dv);
    }
    dv = ev ? dv : 0.0f;
    if constexpr (PSUM) dsum += (double)dv;
    // dy = dout silu(z); dz = dout (y + D x) silu'(z) from the saved pre-gate output
    const float g0 = ev ? T.g.v : 0.0f;
    float dyv = g0;
    if (p.has_z) {
      const float zv = T.z.v, sz = sigmoidf(zv);
      dyv = g0 * (zv * sz);
      if constexpr (!SUM) {
        const float dzv = g0 * T.yp.v * sz * (1.0f + zv * (1.0f - sz));
        if constexpr (UL) {
          buf_store_s<IT>(rdz.rsrc(), offDZ, (uint32_t)(t0 * (int)vdz.s1 * ES), ev && G::lead(lane), dzv);
        } else if (ev && G::lead(lane)) {
          Conv<IT>::store(vpw<IT>(vdz) + b * vdz.s0 + (int64_t)(t0 + tj) * vdz.s1 + (int64_t)(dw + tc) * vdz.s2, dzv);
        }
      }
    }
    const float hstart = k <= 0 ? h0v : T.ck;
    if constexpr (!SUM) {  // the chunk's x and dy rows for the (dB, dC) sums of every wavefront
      xdy[par][0][tj][wv * CW + tc] = xv;
      xdy[par][1][tj][wv * CW + tc] = dyv;
    }
    wave_lds_sync();
    load(T, k - 1);
    // the chunk's B and C rows of this lane's state, read once: the recompute and the walk use
    // them from its first step on
    float rBa[CK], rCa[CK];
    if constexpr (!SUM) lds_row(&S.B[n][0], rBa);
    lds_row(&S.C[n][0], rCa);

    // ------------------------------------------------------------ recompute the chunk's states
    float am[CK], bx[CK], hh[CK + 1];
    if constexpr (!SUM) hh[0] = hstart;
    static_for<0, CK>([&](auto tcst) {
      constexpr int t = decltype(tcst)::value;
      const float dtb = row_bcast<t>(dv);
      float cf;
      if constexpr (M1) {
        am[t] = zoh_am1(dtb, ac);
      } else {
        disc<METHOD>(dtb, ac, am[t], cf);
      }
      if constexpr (!SUM) {
        bx[t] = rBa[t] * row_bcast<t>(xv);
        if constexpr (M1) hh[t + 1] = fmaf(am[t], fmaf(bx[t], ac.invA, hh[t]), hh[t]);
        else hh[t + 1] = fmaf(am[t], hh[t], bcoef<METHOD>(dtb, cf) * bx[t]);
      }
    });

    float dA_acc = 0.0f;
    // ------------------------------------------------------------ walk back, half a chunk at a time
    // The walk broadcasts delta again rather than keeping the recompute's 16 values live (tied
    // to the adjoint: the compiler cannot reuse them).
    float dvw = dv;
    order_after(dvw, lamf);
    static_for_down<0, CK / RH>([&](auto hcst) {
      constexpr int half = decltype(hcst)::value;
      const float *rC = rCa + half * RH, *rB = rBa + half * RH;
      static_for_down<0, RH>([&](auto tcst) {
        constexpr int tt = decltype(tcst)::value;
        constexpr int t = half * RH + tt;
        const float dyb = row_bcast<t>(dyv);
        const float gC = dyb * rC[tt];
        // lambda_t = dy_t C_t + a_{t+1} lambda_{t+1}
        if constexpr (M1) {
          lam += (double)fmaf(m_next, lamf, gC);
        } else {
          lam = fma((double)m_next, lam, (double)gC);
        }
        lamf = (float)lam;
        m_next = am[t];
        if constexpr (SUM) {
          if constexpr (!PSUM) prod *= am[t];
        } else {
          const float dtb = row_bcast<t>(dvw);
          float cf, pD;
          if constexpr (M1) {
            cf = am[t] * ac.invA;
            pD = lamf * fmaf(ac.A, hh[t + 1], bx[t]);  // a (A h_{t-1} + B x) = A h_t + B x
          } else {
            float a_, u_;
            disc<METHOD>(dtb, ac, a_, u_);
            cf = bcoef<METHOD>(dtb, u_);
            if constexpr (METHOD == 1) pD = fmaf(lamf * a_ * ac.A, hh[t], lamf * bx[t]);
            else pD = lamf * (u_ * u_) * fmaf(ac.A, hh[t], bx[t]);
          }
          const float dhc = lamf * cf;
          if constexpr (M1) {
            // A dA = sum_t (dt pD - lambda b): a and b depend on A only through dt A (see k_bwd)
            dA_acc = fmaf(dtb, pD, fmaf(-dhc, bx[t], dA_acc));
          } else {
            // the direct terms, free of that identity's cancellation when dt A is small:
            // Euler d/dA (a h + dt Bx) = dt a h;  bilinear d/dA = dt u^2 (h + dt Bx / 2)
            float a_, u_;
            disc<METHOD>(dtb, ac, a_, u_);
            if constexpr (METHOD == 1) dA_acc = fmaf(lamf * dtb, a_ * hh[t], dA_acc);
            else dA_acc = fmaf(lamf * dtb * (u_ * u_), fmaf(0.5f * dtb, bx[t], hh[t]), dA_acc);
          }
          S.pn[c * WL::PCS + (tt * 2) * WL::NPP + n] = dhc * rB[tt];
          S.pn[c * WL::PCS + (tt * 2 + 1) * WL::NPP + n] = pD;
          pdw[half][tt][0][n][wv * CW + c] = dhc;
          pdw[half][tt][1][n][wv * CW + c] = hh[t + 1];
        }
      });
      if constexpr (!SUM) {
        wave_lds_sync();
        // (dx, ddelta) of step 8 half + j % 8: lane (r, j) sums quantity j / 8 over the states;
        // the previous half's (dB, dC) sums (read during this walk) are formed meanwhile
        {
          float part[NP];
          lds_row(&S.pn[tc * WL::PCS + ((tj % RH) * 2 + tj / RH) * WL::NPP], part);
          dq_flush();
          Rh[half] = pairwise_sum(part);
        }
        // (dB, dC): sum over the workgroup's channels -- the reads now, the sums after the next walk
        lds_barrier();
#pragma unroll
        for (int i = 0; i < IPT; ++i) {
          int item, part;
          red_item(i, item, part);
          const int st = item / (2 * NP), q = (item / NP) % 2, nn = item % NP;
          lds_row(&pdw[half][st][q][nn][part * CPT], dq[i]);
          lds_row(&xdy[par][q][half * RH + st][part * CPT], dqw[i]);
        }
        dq_t = t0 + half * RH;
        dq_L = Lc;
      }
    });
    dA64 += (double)dA_acc;
    if constexpr (SUM) {
      wave_lds_sync();
      return;
    }
    // ------------------------------------------------------------ stores (row-tile lanes)
    // both shifts run with every lane active (a select around a DPP move could otherwise become
    // a masked branch, whose shift would read disabled lanes)
    float sh = row_shr8(Rh[1]), sl = row_shl8(Rh[0]);
    asm volatile("" : "+v"(sh), "+v"(sl));
    const float dxs = tj < RH ? Rh[0] : sh;
    const float dds = tj < RH ? sl : Rh[1];
    const float dxo = fmaf(dyv, dskv, dxs);
    const float ddo = dds * sgv;
    dDp += (double)(dyv * xv);
    dbp += (double)(ev ? ddo : 0.0f);  // padded / inert steps carry state terms but no gradient
    const bool st = ev && G::lead(lane);
    if constexpr (UL) {
      const uint32_t tx_ = (uint32_t)(t0 * (int)vx.s1 * ES);
      buf_store_s<IT>(rdx.rsrc(), offX, tx_, st, dxo);
      buf_store_s<IT>(rddt.rsrc(), offX, tx_, st, ddo);
    } else if (st) {
      const int tg = t0 + tj, dd = dw + tc;
      Conv<IT>::store(vpw<IT>(vdx) + b * vdx.s0 + (int64_t)tg * vdx.s1 + (int64_t)dd * vdx.s2, dxo);
      Conv<IT>::store(vpw<IT>(vddt) + b * vddt.s0 + (int64_t)tg * vddt.s1 + (int64_t)dd * vddt.s2, ddo);
    }
    wave_lds_sync();
  };

  Tiles T0;
  load(T0, k1 - 1);
  chunk(T0, k1 - 1);
  for (int k = k1 - 2; k >= k0 - 1; --k) chunk(T0, k);  // ends on an inert chunk
  if constexpr (!SUM) dq_flush();  // the inert chunk's last half (every store masked)

  // lambda a of the segment's first step (an inert chunk after it already applied it: m_next = 0)
  const double lam_a = M1 ? lam + (double)m_next * lam : lam * (double)m_next;
  const BwdParams &q = params_here<BwdParams>();  // fields read after the loop are loaded here
  if constexpr (SUM) {
    if constexpr (PSUM) prod = fast_exp2((float)((double)ac.A2 * row_sum_f64(dsum)));
    if (dval && nval) {
      ((double *)q.seg_E)[sidx] = lam_a;
      ((float *)q.seg_P)[sidx] = prod;
    }
    return;
  } else {
    if (dval) ((double *)q.ws_dA)[sidx] = M1 ? dA64 * (double)ac.invA : dA64;
    if (q.has_dh0 && dval && nval && seg == 0)
      vstore<float>(q.dh0, b * q.dh0.s0 + d * q.dh0.s1 + n * q.dh0.s2, (float)lam_a);
    // dD and d_bias: the lead row's lanes hold one step slot each; sum them (fixed order)
    const float sD = row_sum((float)dDp), sb = row_sum((float)dbp);
    if (G::lead(lane) && tj == 0 && tval) {
      ((float *)q.ws_dD)[(b * q.nseg + seg) * q.D + dw + tc] = sD;
      ((float *)q.ws_db)[(b * q.nseg + seg) * q.D + dw + tc] = sb;
    }
  }
}

// The adjoint entering each time segment's last step, from the last segment to the first:
// mu[nseg - 1] = dlast (or 0), mu[s - 1] = E[s] + P[s] mu[s]  (float64), one lane per (b, d, n).
template <int NP>
__global__ void __launch_bounds__(kThreads) k_bwd_carry(const BwdParams p) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= p.B * p.D * NP) return;
  const int n = (int)(i % NP);
  const int64_t d = (i / NP) % p.D, b = i / (NP * p.D);
  if (n >= p.N) return;
  double mu = p.has_dlast ? (double)vload<float>(p.dlast, b * p.dlast.s0 + d * p.dlast.s1 + n * p.dlast.s2) : 0.0;
  // the summaries of kCarryGroup segments are read together, then folded in order
  for (int s1 = p.nseg - 1; s1 >= 0; s1 -= kCarryGroup) {
    double Ev[kCarryGroup];
    float Pv[kCarryGroup];
#pragma unroll
    for (int j = 0; j < kCarryGroup; ++j) {  // unconditional reads (a clamped segment is never used)
      const int64_t k = ((b * p.nseg + max(s1 - j, 0)) * p.D + d) * NP + n;
      Ev[j] = ((const double *)p.seg_E)[k];
      Pv[j] = ((const float *)p.seg_P)[k];
    }
#pragma unroll
    for (int j = 0; j < kCarryGroup; ++j) {
      const int s = s1 - j;
      if (s >= 0) {
        ((double *)p.seg_mu)[((b * p.nseg + s) * p.D + d) * NP + n] = mu;
        if (s > 0) mu = Ev[j] + (double)Pv[j] * mu;
      }
    }
  }
}

template <typename IT, int NP, int M, bool SUM, bool LR>
static void bwdw_pass(const BwdParams &p, dim3 grid, hipStream_t s) {
  if (p.uniform) hipLaunchKernelGGL((k_bwdw<IT, NP, M, true, SUM, LR>), grid, dim3(kWave * bwdw_waves(NP)), 0, s, p);
  else hipLaunchKernelGGL((k_bwdw<IT, NP, M, false, SUM, LR>), grid, dim3(kWave * bwdw_waves(NP)), 0, s, p);
}

template <typename IT, int NP, int M, bool LR>
static hipError_t launch_bwdw_lr(const BwdParams &p, hipStream_t s) {
  dim3 grid((unsigned)p.ntiles, (unsigned)(p.B * p.nseg));
  if (p.nseg > 1) {
    bwdw_pass<IT, NP, M, true, LR>(p, grid, s);
    const int64_t lanes = p.B * p.D * NP;
    hipLaunchKernelGGL((k_bwd_carry<NP>), dim3((unsigned)((lanes + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                       p);
  }
  bwdw_pass<IT, NP, M, false, LR>(p, grid, s);
  return hipGetLastError();
}

template <typename IT, int NP, int M>
static hipError_t launch_bwd_t(const BwdParams &p, hipStream_t s) {
  typedef typename Conv<IT>::CT CT;
  if constexpr (sizeof(IT) == 8) {  // float64: the register-staged kernel
    constexpr int WPB = bwd_waves(sizeof(CT), NP);
    constexpr int DT = WPB * (kWave / NP);
    if (p.ntiles != (int)((p.D + DT - 1) / DT) || p.nseg != 1 || p.lowrank) return hipErrorInvalidValue;
    dim3 grid((unsigned)p.ntiles, (unsigned)p.B);
    if (p.uniform) hipLaunchKernelGGL((k_bwd<IT, NP, M, true, false>), grid, dim3(WPB * kWave), 0, s, p);
    else hipLaunchKernelGGL((k_bwd<IT, NP, M, false, false>), grid, dim3(WPB * kWave), 0, s, p);
    return hipGetLastError();
  } else {
    constexpr int DT = bwdw_waves(NP) * (kWave / NP);
    if (p.ntiles != (int)((p.D + DT - 1) / DT)) return hipErrorInvalidValue;
    if constexpr (NP <= 16) {  // the low-rank delta kernels (see launch_fwd)
      if (p.lowrank) return launch_bwdw_lr<IT, NP, M, true>(p, s);
    }
    if (p.lowrank) return hipErrorInvalidValue;
    return launch_bwdw_lr<IT, NP, M, false>(p, s);
  }
}

template <typename IT, int NP>
static hipError_t launch_bwd_m(const BwdParams &p, int method, hipStream_t s) {
  switch (method) {
    case 0: return launch_bwd_t<IT, NP, 0>(p, s);
    case 1: return launch_bwd_t<IT, NP, 1>(p, s);
    default: return launch_bwd_t<IT, NP, 2>(p, s);
  }
}

template <typename IT>
static hipError_t launch_bwd_n(const BwdParams &p, int method, int np, hipStream_t s) {
  if (np != fused_np(p.N, sizeof(IT) == 8 ? 3 : 0)) return hipErrorInvalidValue;
  switch (np) {
    case 8:
      if constexpr (sizeof(IT) == 8) return launch_bwd_m<IT, 8>(p, method, s);
      return hipErrorInvalidValue;
    case 16: return launch_bwd_m<IT, 16>(p, method, s);
    case 32: return launch_bwd_m<IT, 32>(p, method, s);
    default: return launch_bwd_m<IT, 64>(p, method, s);
  }
}

hipError_t launch_bwd(const BwdParams &p, int dtype, int method, int np, hipStream_t s) {
  switch (dtype) {
    case 0: return launch_bwd_n<float>(p, method, np, s);
    case 1: return launch_bwd_n<bf16_t>(p, method, np, s);
    case 2: return launch_bwd_n<f16_t>(p, method, np, s);
    default: return launch_bwd_n<double>(p, method, np, s);
  }
}

hipError_t launch_bwd_finalize(const FinParams &p, int dtype, hipStream_t s) {
  // float partials read as float4 when both partial arrays are 16-byte aligned
  const bool v4 = dtype != 3 && p.np % 4 == 0 && ((uintptr_t)p.ws_dB | (uintptr_t)p.ws_dC) % 16 == 0;
  const int64_t total = fin_bc_lanes(p, v4) + p.D * p.N + p.D;
  dim3 grid((unsigned)((total + 255) / 256));
#define SSM_FIN(OT, CT, V) hipLaunchKernelGGL((k_bwd_finalize<OT, CT, V>), grid, dim3(256), 0, s, p)
  switch (dtype) {
    case 0: if (v4) SSM_FIN(float, float, true); else SSM_FIN(float, float, false); break;
    case 1: if (v4) SSM_FIN(bf16_t, float, true); else SSM_FIN(bf16_t, float, false); break;
    case 2: if (v4) SSM_FIN(f16_t, float, true); else SSM_FIN(f16_t, float, false); break;
    default: SSM_FIN(double, double, false); break;
  }
#undef SSM_FIN
  return hipGetLastError();
}

}  // namespace ssm
