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
#include "ssm_dpp.hpp"
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
// one lane per (b, d, n), segments in order (models/scan.py:160-164 over segments).  The
// summaries of kCarryGroup segments are read together, then folded in order, so the serial
// chain waits for memory once per group instead of once per segment.
template <typename CT, int NP>
__global__ void __launch_bounds__(kThreads) k_fwd_carry(const FwdParams p) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= p.B * p.D * NP) return;
  const int n = (int)(i % NP);
  const int64_t d = (i / NP) % p.D, b = i / (NP * p.D);
  if (n >= p.N) return;
  CT h = p.has_h0 ? vload<CT>(p.h0, b * p.h0.s0 + d * p.h0.s1 + n * p.h0.s2) : (CT)0;
  for (int s0 = 0; s0 < p.nseg; s0 += kCarryGroup) {
    CT Pv[kCarryGroup], Ev[kCarryGroup];
#pragma unroll
    for (int j = 0; j < kCarryGroup; ++j) {  // unconditional reads (a clamped segment is never used)
      const int64_t k = ((b * p.nseg + min(s0 + j, p.nseg - 1)) * p.D + d) * NP + n;
      Pv[j] = ((const CT *)p.seg_P)[k];
      Ev[j] = ((const CT *)p.seg_E)[k];
    }
#pragma unroll
    for (int j = 0; j < kCarryGroup; ++j) {
      if (s0 + j < p.nseg) {
        ((CT *)p.seg_hin)[((b * p.nseg + s0 + j) * p.D + d) * NP + n] = h;
        h = fma(Pv[j], h, Ev[j]);
      }
    }
  }
}

// ------------------------------------------------------------------ float kernels (row tiles)
// The float-compute forward (float32 / bf16 / fp16 inputs, float32 state).  Same mapping and
// chunk walk as k_fwd, with two changes for gfx950's issue model (a wavefront issues at most one
// VALU instruction every few cycles, a dependent one later still, and at B16 D512 N16 only two
// wavefronts share a SIMD):
//   * the per-(step, channel) inputs x, delta and the gate stay in one register per lane (a
//     row tile, ssm_dpp.hpp) and reach each step's lanes by DPP row broadcast, so only B, C
//     and the C h partials pass through LDS;
//   * the chunk loop is software-pipelined: iteration k runs the serial state updates of chunk
//     k - 1 interleaved step by step with the independent per-step work of chunk k (exp,
//     expm1, B x), so most instructions have their operands ready when they issue;
//   * chunks wholly inside the sequence run a copy of the loop body without range selects, and
//     the chunk's inputs are read through windows of the row buffers that start at the chunk
//     (its offset in scalar registers, not one vector add per read).
// The output y_t = sum_n C_t[n] h_t[n] is formed by the lanes that store it: the state lanes
// put h_t itself into LDS and the (step, channel) lane takes the dot product with the step's C
// row (C staged step-major), one FMA per state where a product per state lane and an add
// would be two instructions.
// NP >= 16 (a smaller dstate is padded to 16).
// The states go in channel-major ([c][step_row(t)][n], rows of NPP): a channel block is padded
// by 16 floats, so the two channels of a half-wavefront write 32 distinct banks, and step_row
// orders the rows so that a 16-byte read phase (steps of two channels) hits distinct banks.
template <int NP>
struct FwdwLds {
  static constexpr int CW = kWave / NP, CKP = ck_pad(4), NPP = np_pad(4, NP), YCS = kCK * NPP + 16;
  float B[NP][CKP];
  float Ct[2][kCK][NPP];  // C of the chunk, step-major, one per register set of the pipeline
  float y[CW * YCS];      // the chunk's states h_t at [c * YCS + step_row(t) * NPP + n]
  float lr[kCK][lr_pad(4)];  // low-rank delta input rows of the chunk
  float wr[CW][lr_pad(4)];   // low-rank weight rows of the wavefront's channels
};
constexpr int kFwdwWaves = 4;

// Per-chunk values between the independent phase (iteration k) and the serial phase (k + 1).
template <bool SUM>
struct FwdwStage {
  float m[kCK];  // ZOH: a - 1 (expm1); other methods: a
  float u[kCK];  // ZOH: B x / A; other methods: b
  float x, z;    // the lane's row-tile element of x and the gate
};

template <typename IT, int NP, int METHOD, bool UL, bool SUM, bool LR>
__global__ void __launch_bounds__(kWave * kFwdwWaves) k_fwdw(const FwdParams p) {
  typedef FwdwLds<NP> WL;
  typedef RowGeo<NP> G;
  typedef RowTile<IT, NP, UL> RT;
  typedef FwdwStage<SUM> ST;
  constexpr int CW = G::CW, CK = kCK, WPB = kFwdwWaves;
  __shared__ __align__(16) WL lds_all[WPB];

  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  WL &S = lds_all[wv];
  const int c = lane / NP, n = lane % NP;              // the lane's state h[c][n]
  const int tj = G::step(lane), tc = G::chan(lane);    // the lane's row-tile element (step tj, channel tc)
  const int64_t b = blockIdx.y / p.nseg;
  const int seg = (int)(blockIdx.y % p.nseg);
  if (SUM && seg == p.nseg - 1) return;  // the last segment's summary is never used
  const int k0 = seg * p.seg_chunks;
  const int k1 = k0 + p.seg_chunks < p.nchunks ? k0 + p.seg_chunks : p.nchunks;
  const int dw = (xcd_tile() * WPB + wv) * CW;  // first channel of this wavefront
  const int d = dw + c;
  const bool dval = d < p.D, nval = n < p.N;
  const int L = (int)p.L, D = (int)p.D, N = (int)p.N;
  const bool tval = dw + tc < D;  // the row-tile element's channel exists

  float Av = -1.0f;
  if (dval && nval) {
    Av = vload<float>(p.A, d * p.A.s0 + n * p.A.s1);
    if (p.a_log) Av = -__expf(Av);  // models/mamba.py:81
  }
  const AConst<float> ac = make_aconst(Av);
  float h = 0.0f, prod = 1.0f;
  // Summary pass, ZOH and Euler: the decay product is exp(A sum_t delta_t) -- the lane adds its
  // row-tile delta once per chunk (float64) and the row's 16 lanes are summed at the end,
  // instead of one product per step and state (bilinear keeps the product)
  constexpr bool PSUM = SUM && METHOD != 2;
  double dsum = 0.0;
  const int64_t sidx = ((b * p.nseg + seg) * p.D + d) * NP + n;  // (B, nseg, D, NP) summaries
  if (!SUM && dval && nval) {
    if (p.nseg > kFoldSegs) {
      h = ((const float *)p.seg_hin)[sidx];
    } else {
      // the state entering the segment, folded from the earlier segments' summaries with
      // k_fwd_carry's arithmetic (h <- P h + E); their reads are issued together
      float Pv[kFoldSegs - 1], Ev[kFoldSegs - 1];
#pragma unroll
      for (int s = 0; s < kFoldSegs - 1; ++s) {
        const int64_t k = ((b * p.nseg + s) * p.D + d) * NP + n;
        Pv[s] = s < seg ? ((const float *)p.seg_P)[k] : 0.0f;
        Ev[s] = s < seg ? ((const float *)p.seg_E)[k] : 0.0f;
      }
      if (p.has_h0) h = vload<float>(p.h0, b * p.h0.s0 + d * p.h0.s1 + n * p.h0.s2);
#pragma unroll
      for (int s = 0; s < kFoldSegs - 1; ++s)
        if (s < seg) h = fmaf(Pv[s], h, Ev[s]);
    }
  }
  const float biasv = p.has_bias && tval ? vload<float>(p.bias, (int64_t)(dw + tc) * p.bias.s0) : 0.0f;
  const float dskv = p.has_D && tval ? vload<float>(p.Dsk, (int64_t)(dw + tc) * p.Dsk.s0) : 0.0f;

  const KView vx = p.x, vdt = with_layout<UL>(p.dt, p.x), vz = p.z;  // z keeps its own strides
  const KView vout = with_layout<UL>(p.out, p.x), vB = p.Bm, vC = with_layout<UL>(p.Cm, p.Bm);
  const bool bt = vB.s1 == 1, ctt = vC.s1 == 1;
  const bool zt = p.has_z && p.write_out && !SUM;
  const KView vzl = zt ? vz : vx;  // without a gate the z tile re-reads x (never used)
  struct Tiles {
    RT x, dt, z;
    WaveTile<IT, float, CK, NP, UL> B, C;
    LowRankTile<IT, float, CK> lr;
  };
  constexpr int ES = (int)sizeof(IT), EB = WaveTile<IT, float, CK, NP, UL>::E;
  const uint32_t offX = RT::offset(vx, dw, lane), offZ = RT::offset(vzl, dw, lane);
  uint32_t offB[EB];
  tile_offsets<CK, NP>(offB, vB, 0, bt, lane, ES);
  const __amdgpu_buffer_rsrc_t empty = __builtin_amdgcn_make_buffer_rsrc((void *)p.x.p, (short)0, 0, kBufferFlags);
  // the input rows, read through a window at each chunk (the chunk's offset in scalar registers)
  const RowWin rwx = row_win(vx, b, L, D, ES), rwdt = row_win(LR ? vx : vdt, b, L, D, ES);
  const RowWin rwz = row_win(vzl, b, L, D, ES), rwB = row_win(vB, b, L, N, ES), rwC = row_win(vC, b, L, N, ES);
  __amdgpu_buffer_rsrc_t rblr = empty;
  uint32_t offLR = 0, tstepLR = 0;
  bool rvLR = false;
  if constexpr (LR) {
    rblr = row_buffer(p.dtl, b, L, p.lowrank, ES);
    lowrank_offsets(p.dtl, p.lowrank, lane, ES, offLR, tstepLR, rvLR);
    lowrank_weights<float, CW>(S.wr, p.dtw, p.lowrank, dw, D, lane);
  }
  // Stores of the uniform layout go through buffers over one batch row (the host keeps each
  // below 2^31 bytes): the output, the saved pre-gate output and the chunk states.
  const int64_t ckrow = (int64_t)p.nchunks * p.D * NP;
  const __amdgpu_buffer_rsrc_t rbo = p.write_out ? row_buffer(vout, b, L, D, ES) : empty;
  const __amdgpu_buffer_rsrc_t rby = flat_buffer(p.ypre ? (const float *)p.ypre + b * p.L * p.D : p.x.p,
                                                 p.ypre ? p.L * p.D * 4 : 0);
  const __amdgpu_buffer_rsrc_t rbk = flat_buffer(p.ckpt ? (const float *)p.ckpt + b * ckrow : p.x.p,
                                                 p.ckpt ? ckrow * 4 : 0);
  const uint32_t offO = RT::offset(vout, dw, lane);
  // the saved pre-gate output is (B, D, L) whatever x's layout: 64-byte pieces per wavefront
  const uint32_t offY = (uint32_t)(ypre_index(false, 0, tj, dw + tc, p.L, p.D) * 4);
  const uint32_t tstepY = (uint32_t)(CK * 4);
  const uint32_t offK = (uint32_t)(((int64_t)d * NP + n) * 4);
  // Every load is unconditional (branch-free), two chunks ahead of the chunk being staged; past
  // the segment's end the prefetch re-reads its last chunk.
  auto load = [&](Tiles &T, int k) {
    const int t0 = (k < k1 ? k : k1 - 1) * CK;
    if constexpr (LR) T.lr.load(rblr, offLR + (uint32_t)(t0 * (int)p.dtl.s1 * ES), tstepLR, rvLR);
    if constexpr (UL) {
      const uint32_t tx_ = (uint32_t)(t0 * (int)vx.s1 * ES), tb_ = (uint32_t)(t0 * (int)vB.s1 * ES);
      T.x.load_buf(rwx.at(tx_), offX, 0u);
      if constexpr (!LR) T.dt.load_buf(rwdt.at(tx_), offX, 0u);
      T.B.load_buf(rwB.at(tb_), offB, 0u);
      if (!SUM) T.C.load_buf(rwC.at(tb_), offB, 0u);
      if (!SUM) T.z.load_buf(rwz.at((uint32_t)(t0 * (int)vzl.s1 * ES)), offZ, 0u);
    } else {
      T.x.load(vx, b, t0, L, dw, D, lane);
      if constexpr (!LR) T.dt.load(vdt, b, t0, L, dw, D, lane);
      T.B.load(vB, b, t0, L, 0, N, bt, lane);
      if (!SUM) T.C.load(vC, b, t0, L, 0, N, ctt, lane);
      if (!SUM) T.z.load(vzl, b, t0, L, dw, D, lane);
    }
  };

  // Iteration k: stage chunk k (inert past k1: zero inputs, a = 1, b = 0) and compute its
  // independent per-step values into `nx`, interleaved with the serial updates of chunk k - 1
  // from `pv` (inert before k0); then the outputs of chunk k - 1.  FULL iterations (the
  // caller checks: k0 < k < k1, chunk k wholly inside the sequence, N = NP, every channel of
  // the wavefront real) drop the range selects of the staging and of the stores.
  // Issue priority.  Two wavefronts that share a SIMD would run oldest-first: the older ends
  // several microseconds before the younger, which then runs alone to the end of the launch with
  // its latencies exposed.  Each wavefront instead takes the higher priority in alternate windows
  // of 512 ticks (5.12 us) of the 100 MHz real-time counter, by the parity of its wave slot on the
  // SIMD (HW_ID bits 3:0), so a pair progresses evenly and ends together.
  const unsigned slot_par = __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 4) & 1u;
  auto iter = [&](auto full, auto slot, Tiles &T, int k, ST &pv, ST &nx) {
    constexpr bool F = decltype(full)::value;
    constexpr int SL = decltype(slot)::value;  // the tiles' slot: chunks alternate between the two
    if (((((unsigned)__builtin_amdgcn_s_memrealtime()) >> 9) ^ slot_par) & 1u) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
    const int t0 = k * CK;
    const int Lc = F || k < k1 ? L : 0;
    const bool ev = F || (t0 + tj < Lc && tval);  // the row-tile element is a real (step, channel)
    T.B.template store<!F>(S.B, bt, lane, t0, Lc, 0, N);
    nx.x = ev ? T.x.v : 0.0f;
    nx.z = T.z.v;
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
    if (p.softplus) dv = softplusf(dv);
    dv = ev ? dv : 0.0f;  // padded steps: delta 0 is the identity step
    if constexpr (PSUM) dsum += (double)dv;
    const float xv = nx.x;
    wave_lds_sync();
    // chunk k's C (read by the next iteration's output phase) beside chunk k - 1's (read by
    // this one's, in the other tiles' slot), before the tile registers are refilled
    if (!SUM) T.C.template store_t<!F>(S.Ct[SL], ctt, lane, t0, Lc, 0, N);
    load(T, k + 2);
    float rB[CK];
    lds_row(&S.B[n][0], rB);

    // Scheduling window: step t's independent work follows the update of step t - 2, and the
    // update of step t follows the independent work of step t - 2 (ties, no instructions: the
    // tie on the update rewrites pv.u[t], which no later step reads, so no copy is needed).
    float dvs = dv, xvs = xv, hl1 = h, hl2 = h;
    static_for<0, CK>([&](auto tcst) {
      constexpr int t = decltype(tcst)::value;
      if constexpr (t >= 2) {
        order_after(dvs, hl2);
        order_after(xvs, hl2);
        order_after(pv.u[t], nx.m[t - 2], nx.u[t - 2]);
      }
      // serial update of chunk k - 1 (ZOH: h <- h + (a - 1)(h + B x / A))
      if constexpr (METHOD == 0) {
        h = fmaf(pv.m[t], h + pv.u[t], h);
      } else {
        h = fmaf(pv.m[t], h, pv.u[t]);
        if constexpr (SUM && !PSUM) prod *= pv.m[t];
      }
      if constexpr (!SUM) S.y[c * WL::YCS + step_row(t) * WL::NPP + n] = h;
      // independent values of chunk k
      const float dtb = row_bcast<t>(dvs);
      const float bxr = rB[t] * row_bcast<t>(xvs);
      if constexpr (METHOD == 0) {
        nx.m[t] = zoh_am1(dtb, ac);
        nx.u[t] = bxr * ac.invA;
      } else {
        float coef;
        disc<METHOD>(dtb, ac, nx.m[t], coef);
        nx.u[t] = bcoef<METHOD>(dtb, coef) * bxr;
      }
      hl2 = hl1;
      hl1 = h;
    });
    if constexpr (SUM) {
      wave_lds_sync();
      return;
    }
    const int kp = k - 1;  // the chunk whose outputs are now complete
    const bool live = F || (kp >= k0 && kp < k1);
    wave_lds_sync();
    // outputs of chunk k - 1: the lane of (step tj, channel tc) forms sum_n C[tj][n] h[tj][tc][n]
    // (four interleaved FMA chains, added pairwise)
    float part[NP], cw[NP];
    lds_row(&S.y[tc * WL::YCS + step_row(tj) * WL::NPP], part);
    lds_row(&S.Ct[1 - SL][tj][0], cw);
    const float y = dot_sum(part, cw);
    const int tg = kp * CK + tj, dd = dw + tc;
    const bool st = F ? G::lead(lane) : live && G::lead(lane) && tg < L && tval;
    const float o0 = y + dskv * pv.x;
    const float o = p.has_z ? o0 * (pv.z * sigmoidf(pv.z)) : o0;
    if constexpr (UL) {  // branch-free: masked lanes store out of range (dropped)
      // the chunk's offset is the stores' scalar offset: a masked lane's vector offset lies
      // past every buffer, and the stores of the other lanes lie inside their rows
      const uint32_t kpc = (uint32_t)(F || kp >= 0 ? kp : 0);
      buf_store_s<float>(rbk, offK, kpc * (uint32_t)(p.D * NP * 4), F || (dval && live), h);
      buf_store_s<float>(rby, offY, kpc * tstepY, st, o0);
      buf_store_s<IT>(rbo, offO, kpc * (uint32_t)(CK * (int)vout.s1 * ES), st, o);
    } else {
      if (p.ckpt && dval && live) ((float *)p.ckpt)[((b * p.nchunks + kp) * p.D + d) * NP + n] = h;
      if (st) {
        if (p.ypre) ((float *)p.ypre)[ypre_index(false, b, tg, dd, p.L, p.D)] = o0;
        if (p.write_out) Conv<IT>::store(vpw<IT>(vout) + b * vout.s0 + row_off<UL>(tg, dd, vout.s1, vout.s2), o);
      }
    }
    wave_lds_sync();
  };

  Tiles T0, T1;
  ST P0, P1;
#pragma unroll
  for (int t = 0; t < CK; ++t) {  // inert chunk k0 - 1: a - 1 = 0 (ZOH) / a = 1, b = 0
    P1.m[t] = METHOD == 0 ? 0.0f : 1.0f;
    P1.u[t] = 0.0f;
  }
  P1.x = P1.z = 0.0f;
  load(T0, k0);
  load(T1, k0 + 1);
  const std::integral_constant<bool, false> ranged;
  const std::integral_constant<bool, true> full;
  const std::integral_constant<int, 0> s0;
  const std::integral_constant<int, 1> s1;
  iter(ranged, s0, T0, k0, P1, P0);
  int k = k0 + 1;
  if constexpr (UL) {
    // pairs of whole chunks strictly inside the segment, every lane's state and channel real
    const int kf = min(k1, L / CK);
    if (p.N == NP && p.D % (WPB * CW) == 0) {
      int pairs = 0;  // workgroup-uniform: every wavefront walks the same chunks
      for (; k + 1 < kf; k += 2) {
        iter(full, s1, T1, k, P0, P1);
        iter(full, s0, T0, k + 1, P1, P0);
        if (!SUM && p.sync_pairs && ++pairs == p.sync_pairs) {
          pairs = 0;
          __syncthreads();
        }
      }
    }
  }
  for (; k <= k1; k += 2) {
    iter(ranged, s1, T1, k, P0, P1);
    iter(ranged, s0, T0, k + 1, P1, P0);
  }

  if constexpr (SUM) {
    if constexpr (PSUM) prod = fast_exp2((float)((double)ac.A2 * row_sum_f64(dsum)));
    if (dval && nval) {
      ((float *)p.seg_P)[sidx] = prod;
      ((float *)p.seg_E)[sidx] = h;
    }
  } else if (p.has_last && dval && nval && seg == p.nseg - 1) {
    vstore<float>(p.last, b * p.last.s0 + d * p.last.s1 + n * p.last.s2, h);
  }
}

// ------------------------------------------------------------------ launchers
template <typename IT, int NP, int M, bool SUM, bool LR>
static void fwd_pass(const FwdParams &p, dim3 grid, dim3 block, hipStream_t s) {
  if constexpr (sizeof(IT) == 8) {
    if (p.uniform) hipLaunchKernelGGL((k_fwd<IT, NP, M, true, SUM, LR>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((k_fwd<IT, NP, M, false, SUM, LR>), grid, block, 0, s, p);
  } else {
    if (p.uniform) hipLaunchKernelGGL((k_fwdw<IT, NP, M, true, SUM, LR>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((k_fwdw<IT, NP, M, false, SUM, LR>), grid, block, 0, s, p);
  }
}

template <typename IT, int NP, int M, bool LR>
static hipError_t launch_fwd_t(const FwdParams &p, hipStream_t s) {
  typedef typename Conv<IT>::CT CT;
  constexpr int WPB = sizeof(IT) == 8 ? fwd_waves(sizeof(CT), NP) : kFwdwWaves;
  constexpr int DT = WPB * (kWave / NP);
  dim3 grid((unsigned)((p.D + DT - 1) / DT), (unsigned)(p.B * p.nseg));
  if (p.nseg > 1) {
    fwd_pass<IT, NP, M, true, LR>(p, grid, dim3(WPB * kWave), s);
    if (sizeof(IT) == 8 || p.nseg > kFoldSegs) {  // else the float main pass folds the summaries
      const int64_t lanes = p.B * p.D * NP;
      hipLaunchKernelGGL((k_fwd_carry<CT, NP>), dim3((unsigned)((lanes + kThreads - 1) / kThreads)), dim3(kThreads),
                         0, s, p);
    }
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

// Float compute pads the state to at least 16 (row tiles); float64 keeps 8.
template <typename IT>
static hipError_t launch_fwd_n(const FwdParams &p, int method, int np, hipStream_t s) {
  if (np != fused_np(p.N, sizeof(IT) == 8 ? 3 : 0)) return hipErrorInvalidValue;
  switch (np) {
    case 8:
      if constexpr (sizeof(IT) == 8) return launch_fwd_m<IT, 8>(p, method, s);
      return hipErrorInvalidValue;
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
