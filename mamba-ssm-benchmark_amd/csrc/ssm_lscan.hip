// Linear-recurrence scan algorithms for gfx950: h_t = a_t h_{t-1} + b_t over (B, L, M).
//
// Replaces the four torch scans of models/scan.py with kernels that keep each algorithm's
// structure (so `scan=` still selects an algorithm, as in the reference's SCANS registry,
// models/scan.py:168-173):
//   sequential     models/scan.py:70-76    one lane per (b, m) walks the sequence, reading up
//                                          to 32 steps ahead of the dependent updates.
//   hillis_steele  models/scan.py:87-98    a workgroup owns 64 neighbouring recurrences (lanes
//                                          along m, so every global access is coalesced) and
//                                          runs recursive doubling along time over tiles of 32
//                                          steps (offsets 1, 2 through LDS, 4..16 in
//                                          registers); the state entering a tile is folded
//                                          into its first element (as _fold_h0 does with h0,
//                                          :79-84).
//   blelloch       models/scan.py:101-135  the same 64-recurrence workgroups; up-sweep /
//                                          down-sweep along time over tiles of 64 steps (a
//                                          lane's 16-step block in registers, the block roots
//                                          through LDS), giving exclusive (A, S) prefixes;
//                                          h = a (A h_in + S) + b, the tile's last h carried.
//   chunked        models/scan.py:142-165  three launches: per-chunk summaries from zero
//                                          (P = prod a, E = local end; no states written), a
//                                          scan over the summaries per (b, m) giving each
//                                          chunk's entering state h_in, then each chunk
//                                          scanned from h_in (scan_chunked's local scan plus
//                                          its correction h += P_t h_in, in one pass).
// Direction: with `reverse` the recurrence runs from t = L-1 down to 0.  With `shift` (used
// by the adjoint) the multiplier at a step is the a of the previous step in processing order
// and 1 for the first step: lambda_t = g_t + a_{t+1} lambda_{t+1} (models/scan.py:239-240).
#include "ssm_device.hpp"
#include "ssm_dpp.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"
#include "ssm_wave.hpp"

namespace ssm {

template <typename CT>
struct Chain {
  const LscanParams &P;
  int64_t b, m;
  __device__ __forceinline__ int t_of(int pos) const { return P.reverse ? (int)P.L - 1 - pos : pos; }
  __device__ __forceinline__ CT a_at(int t) const {
    return vload<CT>(P.a, b * P.a.s0 + (int64_t)t * P.a.s1 + m * P.a.s2);
  }
  // multiplier used at processing position pos
  __device__ __forceinline__ CT mult(int pos) const {
    if (!P.shift) return a_at(t_of(pos));
    return pos > 0 ? a_at(t_of(pos - 1)) : (CT)1;
  }
  __device__ __forceinline__ CT b_at(int t) const {
    return vload<CT>(P.b, b * P.b.s0 + (int64_t)t * P.b.s1 + m * P.b.s2);
  }
  __device__ __forceinline__ int64_t h_off(int t) const { return b * P.h.s0 + (int64_t)t * P.h.s1 + m * P.h.s2; }
  __device__ __forceinline__ CT h0() const {
    return P.h0.p ? vload<CT>(P.h0, b * P.h0.s0 + m * P.h0.s1) : (CT)0;
  }
};

// ------------------------------------------------------------------ sequential
// Steps per register set: a lane keeps two sets; while one set's updates run, the reads of the
// other are in flight (512 wavefronts at the bench shape: bytes in flight per wavefront set
// the bandwidth).
template <typename CT> constexpr int seq_ahead() { return sizeof(CT) == 4 ? 32 : 16; }

// One wavefront per workgroup: at (B, M) = (2, 16384) the 512 wavefronts spread over all 256
// CUs (256-lane workgroups would occupy only 128 of them).
constexpr int kSeqThreads = 64;

template <typename CT>
__global__ void __launch_bounds__(kSeqThreads) k_lscan_seq(const LscanParams P) {
  constexpr int K = seq_ahead<CT>();
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.M) return;
  Chain<CT> ch{P, i / P.M, i % P.M};
  const int L = (int)P.L;
  CT h = ch.h0();
  CT a0[K], b0[K], a1[K], b1[K];
  // reads at clamped positions (past the end: re-reads of the last step, never used), so no
  // read waits behind a branch
  auto fetch = [&](CT (&av)[K], CT (&bv)[K], int pos0) {
#pragma unroll
    for (int u = 0; u < K; ++u) {
      const int pos = min(pos0 + u, L - 1);
      av[u] = ch.mult(pos);
      bv[u] = ch.b_at(ch.t_of(pos));
    }
  };
  auto run = [&](const CT (&av)[K], const CT (&bv)[K], int pos0, int n) {
#pragma unroll
    for (int u = 0; u < K; ++u) {
      if (u < n) {
        h = fma(av[u], h, bv[u]);
        vstore<CT>(P.h, ch.h_off(ch.t_of(pos0 + u)), h);
      }
    }
  };
  fetch(a0, b0, 0);
  int pos = 0;
  for (; pos + 2 * K <= L; pos += 2 * K) {
    fetch(a1, b1, pos + K);
    run(a0, b0, pos, K);
    fetch(a0, b0, pos + 2 * K);
    run(a1, b1, pos + K, K);
  }
  if (pos < L) {  // fewer than 2K steps left; a0 holds the next K
    fetch(a1, b1, pos + K);
    run(a0, b0, pos, L - pos);
    run(a1, b1, pos + K, L - pos - K);
  }
}

// Sequential, float, unit stride along m: the same walk with the reads and writes moved through
// LDS tiles.  A wavefront owns 64 consecutive recurrences m of one batch row and walks 16-step
// blocks.  A block's a and b tiles (16 steps x 64 recurrences) are read with 16-byte loads -- a
// lane reads 4 recurrences of one step, so one load instruction carries 4 steps where a read per
// recurrence carries one -- and transposed through LDS so that each lane walks its own
// recurrence; the block's states go back through LDS and leave as 16-byte stores.  With at most
// 63 memory instructions outstanding per wavefront, that puts ~4x the bytes of the one-lane-per-
// recurrence walk in flight.  Reads run kSeqTAhead blocks ahead, at clamped positions (past the
// end: re-reads of the last step, never used).
constexpr int kSeqTB = 16, kSeqTAhead = 3;
typedef float f32x4 __attribute__((ext_vector_type(4)));  // a native vector (HIP's float4 is a struct)

__global__ void __launch_bounds__(64) k_lscan_seqt(const LscanParams P) {
  __shared__ __align__(16) float sA[kSeqTB][64], sB[kSeqTB][64], sH[kSeqTB][64];
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y, m0 = (int64_t)blockIdx.x * 64;
  const int L = (int)P.L;
  const int rl = lane / 16, cl = (lane % 16) * 4;  // the lane's row in a group of 4 steps, its column
  Chain<float> ch{P, b, m0 + lane};
  float h = ch.h0();
  const float *pa = (const float *)P.a.p + b * P.a.s0 + m0 + cl;
  const float *pb = (const float *)P.b.p + b * P.b.s0 + m0 + cl;
  float *ph = (float *)P.h.p + b * P.h.s0 + m0 + cl;
  struct Blk {
    f32x4 a[kSeqTB / 4], b[kSeqTB / 4];
  };
  auto fetch = [&](Blk &k, int pos0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kSeqTB / 4; ++j) {
      const int pos = min(pos0 + rl + 4 * j, L - 1);
      const int apos = P.shift ? max(pos - 1, 0) : pos;  // the shifted multiplier (the adjoint's)
      k.a[j] = *(const f32x4 *)(pa + (int64_t)ch.t_of(apos) * P.a.s1);
      k.b[j] = *(const f32x4 *)(pb + (int64_t)ch.t_of(pos) * P.b.s1);
    }
  };
  auto run = [&](const Blk &k, int pos0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kSeqTB / 4; ++j) {
      *(f32x4 *)&sA[rl + 4 * j][cl] = k.a[j];
      *(f32x4 *)&sB[rl + 4 * j][cl] = k.b[j];
    }
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < kSeqTB; ++r) {
      const float a = (P.shift && pos0 + r == 0) ? 1.0f : sA[r][lane];
      h = fmaf(a, h, sB[r][lane]);
      sH[r][lane] = h;
    }
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < kSeqTB / 4; ++j) {
      const int pos = pos0 + rl + 4 * j;
      const f32x4 v = *(const f32x4 *)&sH[rl + 4 * j][cl];
      if (pos < L) *(f32x4 *)(ph + (int64_t)ch.t_of(pos) * P.h.s1) = v;
    }
    wave_lds_sync();  // the next block's tiles reuse the LDS
  };
  Blk k[kSeqTAhead];
  static_for<0, kSeqTAhead>([&](auto icst) { fetch(k[decltype(icst)::value], decltype(icst)::value * kSeqTB); });
  for (int pos = 0; pos < L; pos += kSeqTAhead * kSeqTB) {
    // blocks past the end are skipped (their reads, clamped, are never used)
    static_for<0, kSeqTAhead>([&](auto icst) {
      constexpr int i = decltype(icst)::value;
      if (pos + i * kSeqTB < L) run(k[i], pos + i * kSeqTB);
      fetch(k[i], pos + (i + kSeqTAhead) * kSeqTB);
    });
  }
}

// The tiled walk's conditions: float, every view with unit stride along m and 16-byte aligned
// rows, M a multiple of 64.
static bool seqt_ok(const LscanParams &P) {
  auto ok = [](const KView &v) {
    return v.s2 == 1 && v.s1 % 4 == 0 && v.s0 % 4 == 0 && ((uintptr_t)v.p % 16) == 0;
  };
  return P.M % 64 == 0 && ok(P.a) && ok(P.b) && ok(P.h);
}

// Tiled parallel scans: a workgroup of 256 lanes owns kScanMC recurrences m (lane % 64) of one
// batch row; lane / 64 selects which time rows of a tile the lane loads, updates and stores.
constexpr int kScanMC = 64, kScanRowLanes = 4;

// ------------------------------------------------------------------ Hillis-Steele
// Recursive doubling over a tile of T = 32 steps: at offset o every step k >= o composes with
// step k - o of the previous pass (models/scan.py:87-98).  Row lane tr holds steps tr, tr + 4,
// ..., so the offsets 4, 8, 16 pair registers of one lane and only the offsets 1 and 2 pair
// different lanes, through LDS.
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_hs(const LscanParams P) {
  constexpr int RL = kScanRowLanes, R = 8, T = RL * R;
  __shared__ CT sA[2][T][kScanMC], sS[2][T][kScanMC], sLast[kScanMC];
  const int mi = threadIdx.x % kScanMC, tr = threadIdx.x / kScanMC;
  const int64_t m = (int64_t)blockIdx.x * kScanMC + mi;
  const bool mval = m < P.M;
  Chain<CT> ch{P, (int64_t)blockIdx.y, mval ? m : 0};
  const int L = (int)P.L;
  CT carry = ch.h0();
  // a tile's inputs are read while the previous tile is scanned
  CT na[R], nb[R];
  auto fetch = [&](int base) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int pos = base + tr + RL * r;
      const bool valid = mval && pos < L;
      na[r] = valid ? ch.mult(pos) : (CT)1;
      nb[r] = valid ? ch.b_at(ch.t_of(pos)) : (CT)0;
    }
  };
  fetch(0);
  for (int base = 0; base < L; base += T) {
    CT A[R], S[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      A[r] = na[r];
      S[r] = nb[r];
    }
    if (tr == 0) S[0] = fma(A[0], carry, S[0]);  // fold the incoming state into the first element
    if (base + T < L) fetch(base + T);
    // offsets 1 and 2 (pass q: o = 2^q) through LDS: step k - o is in row lane tr - o, or in
    // row lane tr - o + 4 one register lower
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int o = 1 << q;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        sA[q][tr + RL * r][mi] = A[r];
        sS[q][tr + RL * r][mi] = S[r];
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int k = tr + RL * r;
        if (k >= o) {
          S[r] = fma(A[r], sS[q][k - o][mi], S[r]);
          A[r] = A[r] * sA[q][k - o][mi];
        }
      }
    }
    // offsets 4, 8, 16 (j = o / 4 registers apart): descending r reads the previous pass's r - j
#pragma unroll
    for (int j = 1; j < R; j *= 2) {
#pragma unroll
      for (int r = R - 1; r >= j; --r) {
        S[r] = fma(A[r], S[r - j], S[r]);
        A[r] = A[r] * A[r - j];
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int pos = base + tr + RL * r;
      if (mval && pos < L) vstore<CT>(P.h, ch.h_off(ch.t_of(pos)), S[r]);
    }
    if (tr == RL - 1) sLast[mi] = S[R - 1];  // step T - 1: the state entering the next tile
    __syncthreads();
    carry = sLast[mi];
  }
}

// ------------------------------------------------------------------ Blelloch
// Up-sweep / down-sweep over a tile of T = 64 steps (models/scan.py:101-135).  Row lane tr
// holds the 16 consecutive steps 16 tr .. 16 tr + 15, so the tree levels of span 2..16 are
// register operations of one lane; the two top levels (span 32, 64) combine the four block
// roots, which every lane of a column reads from LDS and sweeps itself (the same combines in
// every lane, so the same bits).  Each tree node goes through the same combines as in a
// tile-wide sweep.
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_bl(const LscanParams P) {
  constexpr int RL = kScanRowLanes, R = 16, T = RL * R;
  __shared__ CT sRA[RL][kScanMC], sRS[RL][kScanMC], sLast[kScanMC];
  const int mi = threadIdx.x % kScanMC, tr = threadIdx.x / kScanMC;
  const int64_t m = (int64_t)blockIdx.x * kScanMC + mi;
  const bool mval = m < P.M;
  Chain<CT> ch{P, (int64_t)blockIdx.y, mval ? m : 0};
  const int L = (int)P.L;
  CT carry = ch.h0();
  // a tile's inputs are read while the previous tile is scanned
  CT na[R], nb[R];
  auto fetch = [&](int base) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int pos = base + tr * R + r;
      const bool valid = mval && pos < L;
      na[r] = valid ? ch.mult(pos) : (CT)1;  // padding with the identity (1, 0)
      nb[r] = valid ? ch.b_at(ch.t_of(pos)) : (CT)0;
    }
  };
  fetch(0);
  for (int base = 0; base < L; base += T) {
    CT a_own[R], b_own[R], A[R], S[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      a_own[r] = na[r];
      b_own[r] = nb[r];
      A[r] = na[r];
      S[r] = nb[r];
    }
    if (base + T < L) fetch(base + T);
    // up-sweep inside the lane's block: right <- right o left at nodes (j + 1) s - 1
#pragma unroll
    for (int sp = 2; sp <= R; sp *= 2) {
#pragma unroll
      for (int k = sp - 1; k < R; k += sp) {
        const int l = k - sp / 2;
        S[k] = fma(A[k], S[l], S[k]);
        A[k] = A[k] * A[l];
      }
    }
    sRA[tr][mi] = A[R - 1];
    sRS[tr][mi] = S[R - 1];
    __syncthreads();
    // the two top levels over the block roots (nodes 1, 3 at span 2; node 3 at span 4), the
    // root set to the identity, then their down-sweep: each root becomes the composition of
    // the blocks before it
    CT rA[RL], rS[RL];
#pragma unroll
    for (int q = 0; q < RL; ++q) {
      rA[q] = sRA[q][mi];
      rS[q] = sRS[q][mi];
    }
#pragma unroll
    for (int sp = 2; sp <= RL; sp *= 2) {
#pragma unroll
      for (int k = sp - 1; k < RL; k += sp) {
        const int l = k - sp / 2;
        rS[k] = fma(rA[k], rS[l], rS[k]);
        rA[k] = rA[k] * rA[l];
      }
    }
    rA[RL - 1] = 1;
    rS[RL - 1] = 0;
#pragma unroll
    for (int sp = RL; sp >= 2; sp /= 2) {
#pragma unroll
      for (int k = sp - 1; k < RL; k += sp) {
        const int l = k - sp / 2;
        const CT tA = rA[l], tS = rS[l];
        rA[l] = rA[k];
        rS[l] = rS[k];
        rS[k] = fma(rS[k], tA, tS);
        rA[k] = rA[k] * tA;
      }
    }
    A[R - 1] = rA[tr];
    S[R - 1] = rS[tr];
    // down-sweep inside the block: left <- right; right <- left_old o right
#pragma unroll
    for (int sp = R; sp >= 2; sp /= 2) {
#pragma unroll
      for (int k = sp - 1; k < R; k += sp) {
        const int l = k - sp / 2;
        const CT tA = A[l], tS = S[l];
        A[l] = A[k];
        S[l] = S[k];
        S[k] = fma(S[k], tA, tS);
        A[k] = A[k] * tA;
      }
    }
    // exclusive prefixes: the state entering step k is A_k h_in + S_k
    CT h = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int pos = base + tr * R + r;
      h = fma(a_own[r], fma(A[r], carry, S[r]), b_own[r]);
      if (mval && pos < L) vstore<CT>(P.h, ch.h_off(ch.t_of(pos)), h);
    }
    if (tr == RL - 1) sLast[mi] = h;  // step T - 1: the state entering the next tile
    __syncthreads();
    carry = sLast[mi];
  }
}

// ------------------------------------------------------------------ chunked (three phases)
// Reduce, carry, scan: each chunk's summary (P = product of its multipliers, E = its end
// state from zero) is formed without writing any state; a sequential scan over the summaries
// gives every chunk's entering state h_in; each chunk is then scanned from h_in.  The chunks'
// states equal scan_chunked's local states corrected by P_t h_in (models/scan.py:152-164),
// to rounding, and the states are written once instead of written, re-read and rewritten.
constexpr int kSeqAhead = 16;  // steps whose inputs are read before their dependent updates

// Walks positions [p0, p1) of a chain from state h: h <- mult h + b at each step, with the
// product of the multipliers in prod (REDUCE) or every state stored (otherwise).
template <typename CT, bool REDUCE>
__device__ __forceinline__ void chunk_walk(const LscanParams &P, const Chain<CT> &ch, int p0, int p1, CT &h,
                                           CT &prod) {
  int pos = p0;
  for (; pos + kSeqAhead <= p1; pos += kSeqAhead) {  // inputs read ahead of the updates
    CT av[kSeqAhead], bv[kSeqAhead];
#pragma unroll
    for (int u = 0; u < kSeqAhead; ++u) {
      av[u] = ch.mult(pos + u);
      bv[u] = ch.b_at(ch.t_of(pos + u));
    }
#pragma unroll
    for (int u = 0; u < kSeqAhead; ++u) {
      h = fma(av[u], h, bv[u]);
      if constexpr (REDUCE) prod *= av[u];
      else vstore<CT>(P.h, ch.h_off(ch.t_of(pos + u)), h);
    }
  }
  for (; pos < p1; ++pos) {
    const CT a = ch.mult(pos);
    h = fma(a, h, ch.b_at(ch.t_of(pos)));
    if constexpr (REDUCE) prod *= a;
    else vstore<CT>(P.h, ch.h_off(ch.t_of(pos)), h);
  }
}

template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_chunk_reduce(const LscanParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.nc * P.M) return;
  const int64_t m = i % P.M, cj = (i / P.M) % P.nc, b = i / (P.M * P.nc);
  Chain<CT> ch{P, b, m};
  const int p0 = (int)cj * P.chunk;
  const int p1 = p0 + P.chunk < (int)P.L ? p0 + P.chunk : (int)P.L;
  CT h = 0, prod = 1;
  chunk_walk<CT, true>(P, ch, p0, p1, h, prod);
  CT *ws = (CT *)P.ws;
  const int64_t stride = P.B * P.nc * P.M;
  ws[i] = prod;        // P: product of the chunk's multipliers
  ws[stride + i] = h;  // E: end state from zero
}

template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_chunk_carry(const LscanParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.M) return;
  const int64_t m = i % P.M, b = i / P.M;
  Chain<CT> ch{P, b, m};
  CT *ws = (CT *)P.ws;
  const int64_t stride = P.B * P.nc * P.M;
  CT hin = ch.h0();
  // the summaries of kCarryGroup chunks are read together (unconditionally: a clamped chunk is
  // never used), then folded in order
  for (int c0 = 0; c0 < P.nc; c0 += kCarryGroup) {
    CT Pv[kCarryGroup], Ev[kCarryGroup];
#pragma unroll
    for (int j = 0; j < kCarryGroup; ++j) {
      const int64_t k = (b * P.nc + min((int64_t)(c0 + j), P.nc - 1)) * P.M + m;
      Pv[j] = ws[k];
      Ev[j] = ws[stride + k];
    }
#pragma unroll
    for (int j = 0; j < kCarryGroup; ++j) {
      if (c0 + j < P.nc) {
        ws[2 * stride + (b * P.nc + c0 + j) * P.M + m] = hin;  // state entering chunk c0 + j
        hin = fma(Pv[j], hin, Ev[j]);
      }
    }
  }
}

template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_chunk_scan(const LscanParams P) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P.B * P.nc * P.M) return;
  const int64_t m = i % P.M, cj = (i / P.M) % P.nc, b = i / (P.M * P.nc);
  Chain<CT> ch{P, b, m};
  const int p0 = (int)cj * P.chunk;
  const int p1 = p0 + P.chunk < (int)P.L ? p0 + P.chunk : (int)P.L;
  CT h = ((const CT *)P.ws)[2 * P.B * P.nc * P.M + i], prod = 1;
  chunk_walk<CT, false>(P, ch, p0, p1, h, prod);
}

// ------------------------------------------------------------------ adjoint epilogue
// da_t = lambda_t * h_prev(t), dh0 = a_first * lambda_first (first in the forward's order).
template <typename CT>
__device__ __forceinline__ void lscan_grad_at(const LscanGradParams &P, int64_t b, int64_t t, int64_t m) {
  const CT lam = vload<CT>(P.db, b * P.db.s0 + t * P.db.s1 + m * P.db.s2);
  const int64_t tp = P.reverse ? t + 1 : t - 1;  // previous step of the forward scan
  CT hp;
  if (tp >= 0 && tp < P.L) hp = vload<CT>(P.h, b * P.h.s0 + tp * P.h.s1 + m * P.h.s2);
  else hp = P.h0.p ? vload<CT>(P.h0, b * P.h0.s0 + m * P.h0.s1) : (CT)0;
  vstore<CT>(P.da, b * P.da.s0 + t * P.da.s1 + m * P.da.s2, lam * hp);
  const int64_t tfirst = P.reverse ? P.L - 1 : 0;
  if (t == tfirst && P.dh0.p)
    vstore<CT>(P.dh0, b * P.dh0.s0 + m * P.dh0.s1,
               vload<CT>(P.a, b * P.a.s0 + t * P.a.s1 + m * P.a.s2) * lam);
}

// grid: x over m (256 lanes), y over t, z over b; each strides over t and b past 65535
template <typename CT>
__global__ void __launch_bounds__(256) k_lscan_grad(const LscanGradParams P) {
  const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= P.M) return;
  for (int64_t b = blockIdx.z; b < P.B; b += gridDim.z)
    for (int64_t t = blockIdx.y; t < P.L; t += gridDim.y) lscan_grad_at<CT>(P, b, t, m);
}


template <typename CT>
static hipError_t launch_lscan_t(const LscanParams &P, int algo, hipStream_t s) {
  const int64_t chains = P.B * P.M;
  switch (algo) {
    case 1:
      if (sizeof(CT) == 4 && seqt_ok(P)) {
        hipLaunchKernelGGL(k_lscan_seqt, dim3((unsigned)(P.M / 64), (unsigned)P.B), dim3(64), 0, s, P);
        break;
      }
      hipLaunchKernelGGL((k_lscan_seq<CT>), dim3((unsigned)((chains + kSeqThreads - 1) / kSeqThreads)),
                         dim3(kSeqThreads), 0, s, P);
      break;
    case 2:
      hipLaunchKernelGGL((k_lscan_hs<CT>), dim3((unsigned)((P.M + kScanMC - 1) / kScanMC), (unsigned)P.B), dim3(256),
                         0, s, P);
      break;
    case 3:
      hipLaunchKernelGGL((k_lscan_bl<CT>), dim3((unsigned)((P.M + kScanMC - 1) / kScanMC), (unsigned)P.B), dim3(256),
                         0, s, P);
      break;
    default: {
      const int64_t n = P.B * P.nc * P.M;
      hipLaunchKernelGGL((k_lscan_chunk_reduce<CT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, P);
      hipLaunchKernelGGL((k_lscan_chunk_carry<CT>), dim3((unsigned)((chains + 255) / 256)), dim3(256), 0, s, P);
      hipLaunchKernelGGL((k_lscan_chunk_scan<CT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, P);
    }
  }
  return hipGetLastError();
}

hipError_t launch_lscan(const LscanParams &P, int algo, int dtype, hipStream_t s) {
  return dtype == 3 ? launch_lscan_t<double>(P, algo, s) : launch_lscan_t<float>(P, algo, s);
}

hipError_t launch_lscan_grad(const LscanGradParams &P, int dtype, hipStream_t s) {
  dim3 grid((unsigned)((P.M + 255) / 256), (unsigned)(P.L < 65535 ? P.L : 65535), (unsigned)(P.B < 65535 ? P.B : 65535));
  if (dtype == 3) hipLaunchKernelGGL((k_lscan_grad<double>), grid, dim3(256), 0, s, P);
  else hipLaunchKernelGGL((k_lscan_grad<float>), grid, dim3(256), 0, s, P);
  return hipGetLastError();
}

}  // namespace ssm
