// Fused selective-scan forward for gfx950.
//
// Replaces kernels/triton_scan.py:27-74 (_fwd_kernel) and :83-140 (_fwd_chunked_kernel) and
// the forward of models/scan.py:202-217; the D skip and SiLU gate of models/mamba.py:124 (and
// an optional delta bias + softplus, models/mamba.py:76) are fused.
//
// Mapping: one lane per (channel, state).  Each 64-lane wavefront owns CW = 64/NP channels
// of one batch row and walks time in chunks of CK steps, entirely on its own (no workgroup
// barrier: at B16 D512 N16 only 2 wavefronts share a SIMD, and barriers would idle it).
// Per chunk a wavefront
//   1. stores into its private LDS region the chunk's x, delta (bias/softplus applied) for
//      its channels and B, C for all states -- loaded into registers one chunk ahead with
//      coalesced reads along whichever of L / D has unit stride;
//   2. runs the CK recurrence steps per lane in register batches of RB steps: a batch's
//      inputs come from 16-byte LDS reads (the next batch is read before the current one is
//      computed), its a_t and b_t are formed independently, then the RB dependent h-updates
//      run back to back; each C_t h_t partial goes to LDS;
//   3. sums the partials over the NP states with (t, channel)-mapped lanes, applies the skip
//      and gate and stores the outputs (coalesced); saves the chunk-end state, and the
//      pre-gate output when there is a gate, if the backward needs them.
//
// Long sequences (few batch rows x channels, e.g. B1 D512 at L = 131072) are split into time
// segments so that enough wavefronts exist: the two-level structure of scan_chunked
// (models/scan.py:142-165) with segments in place of chunks.  A summary pass (SUM = true)
// walks each segment from a zero state, skipping C and the outputs, and keeps the product of
// its decays; a carry kernel scans the (product, end state) pairs per (b, d, n); the main pass
// then restarts every segment from the state that enters it.
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"
#include "ssm_wave.hpp"

namespace ssm {

template <typename CT, int NP>
struct FwdWaveLds {
  static constexpr int CW = kWave / NP, CK = kCK, CKP = ck_pad((int)sizeof(CT));
  CT x[CW][CKP];
  CT dt[CW][CKP];
  CT B[NP][CKP];
  CT C[NP][CKP];
  CT y[CK][CW][np_pad((int)sizeof(CT), NP)];
  CT lr[CK][lr_pad((int)sizeof(CT))];  // low-rank delta input rows of the chunk
  CT wr[CW][lr_pad((int)sizeof(CT))];  // low-rank weight rows of the wavefront's channels
};

template <typename IT, int NP, int METHOD, bool UL, bool SUM, bool LR>
__global__ void __launch_bounds__(kWave * fwd_waves(sizeof(typename Conv<IT>::CT), NP))
k_fwd(const FwdParams p) {
  typedef typename Conv<IT>::CT CT;
  typedef FwdWaveLds<CT, NP> WL;
  constexpr int CW = WL::CW, CK = WL::CK;
  constexpr int WPB = fwd_waves(sizeof(CT), NP);
  constexpr int RB = 32 / (int)sizeof(CT) > CK ? CK : 32 / (int)sizeof(CT);  // register batch
  static_assert(sizeof(WL) == fwd_wave_bytes(sizeof(CT), NP), "LDS layout");
  __shared__ __align__(16) WL lds_all[WPB];

  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  WL &S = lds_all[wv];
  const int c = lane / NP, n = lane % NP;
  const int64_t b = blockIdx.y / p.nseg;
  const int seg = (int)(blockIdx.y % p.nseg);
  const int k0 = seg * p.seg_chunks;
  const int k1 = k0 + p.seg_chunks < p.nchunks ? k0 + p.seg_chunks : p.nchunks;
  const int dw = (blockIdx.x * WPB + wv) * CW;  // first channel of this wavefront
  const int d = dw + c;
  const bool dval = d < p.D, nval = n < p.N;
  const int L = (int)p.L, D = (int)p.D, N = (int)p.N;

  CT Av = (CT)-1;
  if (dval && nval) {
    Av = vload<CT>(p.A, d * p.A.s0 + n * p.A.s1);
    if (p.a_log) Av = -exp(Av);  // models/mamba.py:81
  }
  const AConst<CT> ac = make_aconst(Av);
  CT h = 0, prod = 1;
  const int64_t sidx = ((b * p.nseg + seg) * p.D + d) * NP + n;  // (B, nseg, D, NP) summaries
  if (!SUM && dval && nval) {
    if (p.nseg > 1) h = ((const CT *)p.seg_hin)[sidx];
    else if (p.has_h0) h = vload<CT>(p.h0, b * p.h0.s0 + d * p.h0.s1 + n * p.h0.s2);
  }

  const KView vx = p.x, vdt = with_layout<UL>(p.dt, p.x), vz = p.z;  // z keeps its own strides
  const KView vout = with_layout<UL>(p.out, p.x), vB = p.Bm, vC = with_layout<UL>(p.Cm, p.Bm);
  const bool xt = vx.s1 == 1, dtt = vdt.s1 == 1, bt = vB.s1 == 1, ctt = vC.s1 == 1;
  const bool ot = vout.s1 == 1;
  // Global reads run two chunks ahead of the compute: tiles ping-pong between two register
  // sets, and a set is refilled (chunk k + 2) as soon as its chunk is staged in LDS.
  const bool zt = p.has_z && p.write_out && !SUM;
  struct Tiles {
    WaveTile<IT, CT, CK, CW, UL> x, dt, z;
    WaveTile<IT, CT, CK, NP, UL> B, C;
    LowRankTile<IT, CT, CK> lr;
  };
  CT biasv[WaveTile<IT, CT, CK, CW, UL>::E], dskv[WaveTile<IT, CT, CK, CW, UL>::E];
  tile_bias<CT, CK, CW>(biasv, p.has_bias, p.bias, dw, D, dtt, lane);
  tile_bias<CT, CK, CW>(dskv, p.has_D, p.Dsk, dw, D, ot, lane);  // D skip in the output mapping
  // Every load is unconditional (no branch around it) so that waiting for one chunk's tiles
  // leaves the next chunk's loads and earlier stores in flight; past the segment's end the
  // prefetch re-reads its last chunk, and without a gate the z tile reads x.
  const KView vzl = zt ? vz : vx;
  // With a uniform layout x, delta, z share one set of lane offsets (and B, C another) and are
  // read through raw buffers; otherwise through clamped global addresses.
  constexpr int ES = (int)sizeof(IT);
  constexpr int EX = WaveTile<IT, CT, CK, CW, UL>::E, EB = WaveTile<IT, CT, CK, NP, UL>::E;
  uint32_t offX[EX], offB[EB], offZ[EX];
  tile_offsets<CK, CW>(offX, vx, dw, xt, lane, ES);
  tile_offsets<CK, NP>(offB, vB, 0, bt, lane, ES);
  tile_offsets<CK, CW>(offZ, vzl, dw, ot, lane, ES);  // the gate (e.g. the in_proj split) may differ
  const __amdgpu_buffer_rsrc_t empty = __builtin_amdgcn_make_buffer_rsrc((void *)p.x.p, (short)0, 0, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rbx = row_buffer(vx, b, L, D, ES);
  const __amdgpu_buffer_rsrc_t rbdt = LR ? empty : row_buffer(vdt, b, L, D, ES);
  const __amdgpu_buffer_rsrc_t rbz = row_buffer(vzl, b, L, D, ES);
  const __amdgpu_buffer_rsrc_t rbB = row_buffer(vB, b, L, N, ES), rbC = row_buffer(vC, b, L, N, ES);
  // low-rank delta: input block reads and the weight rows in LDS
  __amdgpu_buffer_rsrc_t rblr = empty;
  uint32_t offLR = 0, tstepLR = 0;
  bool rvLR = false;
  if constexpr (LR) {
    rblr = row_buffer(p.dtl, b, L, p.lowrank, ES);
    lowrank_offsets(p.dtl, p.lowrank, lane, ES, offLR, tstepLR, rvLR);
    lowrank_weights<CT, CW>(S.wr, p.dtw, p.lowrank, dw, D, lane);
  }
  auto load = [&](Tiles &T, int k) {
    const int t0 = (k < k1 ? k : k1 - 1) * CK;
    if constexpr (LR) T.lr.load(rblr, offLR + (uint32_t)(t0 * (int)p.dtl.s1 * ES), tstepLR, rvLR);
    if constexpr (UL) {
      const uint32_t tx_ = (uint32_t)(t0 * (int)vx.s1 * ES), tb_ = (uint32_t)(t0 * (int)vB.s1 * ES);
      T.x.load_buf(rbx, offX, tx_);
      T.dt.load_buf(rbdt, offX, tx_);
      T.B.load_buf(rbB, offB, tb_);
      if (!SUM) T.C.load_buf(rbC, offB, tb_);
      if (!SUM) T.z.load_buf(rbz, offZ, (uint32_t)(t0 * (int)vzl.s1 * ES));
    } else {
      T.x.load(vx, b, t0, L, dw, D, xt, lane);
      T.dt.load(vdt, b, t0, L, dw, D, dtt, lane);
      T.B.load(vB, b, t0, L, 0, N, bt, lane);
      if (!SUM) T.C.load(vC, b, t0, L, 0, N, ctt, lane);
      if (!SUM) T.z.load(vzl, b, t0, L, dw, D, ot, lane);  // the output phase's (t, channel) mapping
    }
  };
  // A chunk k >= k1 is inert: its staged inputs are all zero (a = 1, b = 0 leaves h unchanged)
  // and it stores nothing, so chunks always run in pairs and the loop is entered with the
  // same loads and stores in flight as on its back edge.
  auto chunk = [&](Tiles &T, int k) {
    const int t0 = k * CK;
    const int Lc = k < k1 ? L : 0;  // time bound of this chunk's elements
    T.x.store(S.x, xt, lane, t0, Lc, dw, D);
    if constexpr (LR) {
      T.lr.store(S.lr, lane);
      wave_lds_sync();
      lowrank_delta<IT, CT, CK, CW, UL>(T.dt, S.lr, S.wr, dtt, lane);
    }
    store_delta_w<IT, CT, CK, CW, WL::CKP, UL>(T.dt, S.dt, nullptr, dtt, lane, p.softplus, biasv, dw, D, t0, Lc);
    T.B.store(S.B, bt, lane, t0, Lc, 0, N);
    if (!SUM) T.C.store(S.C, ctt, lane, t0, Lc, 0, N);
    CT zv[WaveTile<IT, CT, CK, CW, UL>::E];
#pragma unroll
    for (int i = 0; i < WaveTile<IT, CT, CK, CW, UL>::E; ++i) zv[i] = T.z.v[i];
    wave_lds_sync();
    load(T, k + 2);

    CT rdt[RB], rx[RB], rB[RB], rC[RB];
    lds_row(&S.dt[c][0], rdt);
    lds_row(&S.x[c][0], rx);
    lds_row(&S.B[n][0], rB);
    if (!SUM) lds_row(&S.C[n][0], rC);
#pragma unroll
    for (int q = 0; q < CK / RB; ++q) {
      CT ndt[RB], nx[RB], nB[RB], nC[RB];
      if (q + 1 < CK / RB) {
        lds_row(&S.dt[c][(q + 1) * RB], ndt);
        lds_row(&S.x[c][(q + 1) * RB], nx);
        lds_row(&S.B[n][(q + 1) * RB], nB);
        if (!SUM) lds_row(&S.C[n][(q + 1) * RB], nC);
      }
      // ZOH keeps a - 1 (accurate expm1) and, with b = (a - 1) Bx / A, updates
      // h <- h + (a - 1)(h + Bx / A): the decay keeps its relative accuracy for slowly
      // decaying states (a close to 1), and b needs no separate coefficient.
      CT a[RB], bx[RB];
#pragma unroll
      for (int tt = 0; tt < RB; ++tt) {
        if constexpr (METHOD == 0) {
          a[tt] = zoh_am1(rdt[tt], ac);
          bx[tt] = (rB[tt] * rx[tt]) * ac.invA;
        } else {
          CT coef;
          disc<METHOD>(rdt[tt], ac, a[tt], coef);
          bx[tt] = bcoef<METHOD>(rdt[tt], coef) * (rB[tt] * rx[tt]);
        }
      }
#pragma unroll
      for (int tt = 0; tt < RB; ++tt) {
        if constexpr (METHOD == 0) h = fma(a[tt], h + bx[tt], h);
        else h = fma(a[tt], h, bx[tt]);
        if constexpr (SUM) {  // padded steps (t >= L) have delta 0, i.e. a = 1, b = 0
          if constexpr (METHOD == 0) prod = fma(a[tt], prod, prod);
          else prod *= a[tt];
        } else {
          S.y[q * RB + tt][c][n] = rC[tt] * h;
        }
      }
      if (q + 1 < CK / RB) {
#pragma unroll
        for (int j = 0; j < RB; ++j) {
          rdt[j] = ndt[j];
          rx[j] = nx[j];
          rB[j] = nB[j];
          if (!SUM) rC[j] = nC[j];
        }
      }
    }
    if constexpr (SUM) {
      wave_lds_sync();
      return;
    }
    if (p.ckpt && dval && k < k1)
      ((CT *)p.ckpt)[((b * p.nchunks + k) * p.D + d) * NP + n] = h;
    wave_lds_sync();

    // outputs: sum over states, (y + D x) * silu(z), coalesced along the output's unit axis
#pragma unroll
    for (int i = 0; i < (CK * CW + kWave - 1) / kWave; ++i) {
      const int e = lane + i * kWave;
      if (e >= CK * CW) break;
      int t, cc;
      tc_of<CK, CW>(e, ot, t, cc);
      const int tg = t0 + t, dd = dw + cc;
      CT part[NP];
      lds_row(&S.y[t][cc][0], part);
      const CT xv = S.x[cc][t];  // read with the partials: one LDS round trip
      CT y = 0;
#pragma unroll
      for (int j = 0; j < NP; ++j) y += part[j];
      if (tg >= Lc || dd >= D) continue;
      const CT skip = p.has_D ? dskv[i] * xv : (CT)0;
      if (p.ypre) ((CT *)p.ypre)[ypre_index(!xt, b, tg, dd, p.L, p.D)] = y + skip;
      if (!p.write_out) continue;
      CT o = y + skip;
      if (p.has_z) o *= zv[i] * sigmoid_ct<CT>(zv[i]);
      Conv<IT>::store(vpw<IT>(vout) + b * vout.s0 + row_off<UL>(tg, dd, vout.s1, vout.s2), o);
    }
    wave_lds_sync();
  };

  Tiles T0, T1;
  load(T0, k0);
  load(T1, k0 + 1);
  chunk(T0, k0);
  chunk(T1, k0 + 1);
  for (int k = k0 + 2; k < k1; k += 2) {
    chunk(T0, k);
    chunk(T1, k + 1);
  }

  if constexpr (SUM) {
    if (dval && nval) {
      ((CT *)p.seg_P)[sidx] = prod;
      ((CT *)p.seg_E)[sidx] = h;
    }
  } else if (p.has_last && dval && nval && seg == p.nseg - 1) {
    vstore<CT>(p.last, b * p.last.s0 + d * p.last.s1 + n * p.last.s2, h);
  }
}

// State entering each time segment: h_in[0] = h0 (or 0), h_in[s+1] = P[s] h_in[s] + E[s],
// one lane per (b, d, n), segments in order (models/scan.py:160-164 over segments).
template <typename CT, int NP>
__global__ void __launch_bounds__(kThreads) k_fwd_carry(const FwdParams p) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= p.B * p.D * NP) return;
  const int n = (int)(i % NP);
  const int64_t d = (i / NP) % p.D, b = i / (NP * p.D);
  if (n >= p.N) return;
  CT h = p.has_h0 ? vload<CT>(p.h0, b * p.h0.s0 + d * p.h0.s1 + n * p.h0.s2) : (CT)0;
  for (int s = 0; s < p.nseg; ++s) {
    const int64_t k = ((b * p.nseg + s) * p.D + d) * NP + n;
    ((CT *)p.seg_hin)[k] = h;
    h = fma(((const CT *)p.seg_P)[k], h, ((const CT *)p.seg_E)[k]);
  }
}

template <typename IT, int NP, int M, bool SUM, bool LR>
static void fwd_pass(const FwdParams &p, dim3 grid, dim3 block, hipStream_t s) {
  if (p.uniform) hipLaunchKernelGGL((k_fwd<IT, NP, M, true, SUM, LR>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((k_fwd<IT, NP, M, false, SUM, LR>), grid, block, 0, s, p);
}

template <typename IT, int NP, int M, bool LR>
static hipError_t launch_fwd_t(const FwdParams &p, hipStream_t s) {
  typedef typename Conv<IT>::CT CT;
  constexpr int WPB = fwd_waves(sizeof(CT), NP);
  constexpr int DT = WPB * (kWave / NP);
  dim3 grid((unsigned)((p.D + DT - 1) / DT), (unsigned)(p.B * p.nseg));
  if (p.nseg > 1) {
    fwd_pass<IT, NP, M, true, LR>(p, grid, dim3(WPB * kWave), s);
    const int64_t lanes = p.B * p.D * NP;
    hipLaunchKernelGGL((k_fwd_carry<CT, NP>), dim3((unsigned)((lanes + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       s, p);
  }
  fwd_pass<IT, NP, M, false, LR>(p, grid, dim3(WPB * kWave), s);
  return hipGetLastError();
}

// The low-rank delta kernels exist for dstate <= 16 and 16/32-bit inputs (the ABI rejects the
// other combinations).
template <typename IT, int NP, int M>
static hipError_t launch_fwd_lr(const FwdParams &p, hipStream_t s) {
  if constexpr (NP <= 16 && sizeof(IT) <= 4) {
    if (p.lowrank) return launch_fwd_t<IT, NP, M, true>(p, s);
  }
  if (p.lowrank) return hipErrorInvalidValue;
  return launch_fwd_t<IT, NP, M, false>(p, s);
}

template <typename IT, int NP>
static hipError_t launch_fwd_m(const FwdParams &p, int method, hipStream_t s) {
  switch (method) {
    case 0: return launch_fwd_lr<IT, NP, 0>(p, s);
    case 1: return launch_fwd_lr<IT, NP, 1>(p, s);
    default: return launch_fwd_lr<IT, NP, 2>(p, s);
  }
}

template <typename IT>
static hipError_t launch_fwd_n(const FwdParams &p, int method, int np, hipStream_t s) {
  switch (np) {
    case 8: return launch_fwd_m<IT, 8>(p, method, s);
    case 16: return launch_fwd_m<IT, 16>(p, method, s);
    case 32: return launch_fwd_m<IT, 32>(p, method, s);
    default: return launch_fwd_m<IT, 64>(p, method, s);
  }
}

hipError_t launch_fwd(const FwdParams &p, int dtype, int method, int np, hipStream_t s) {
  switch (dtype) {
    case 0: return launch_fwd_n<float>(p, method, np, s);
    case 1: return launch_fwd_n<bf16_t>(p, method, np, s);
    case 2: return launch_fwd_n<f16_t>(p, method, np, s);
    default: return launch_fwd_n<double>(p, method, np, s);
  }
}

}  // namespace ssm
