// Parameter blocks and launcher declarations shared by the C ABI (ssm_abi.cpp) and the
// kernel translation units.  Plain structs: they are passed to kernels by value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssm {

struct KView {
  const void *p;
  int64_t s0, s1, s2;
};

// Geometry of the fused kernels.  A wavefront owns 64/NP channels x NP states; CK time steps
// are staged per chunk, and the state at the end of every chunk is what the forward saves for
// the backward.  Waves per workgroup are chosen so the per-wave LDS regions fit in 64 KiB.
constexpr int kCK = 16;
constexpr int kFoldSegs = 8;     // time segments the forward's main pass folds without a carry pass
constexpr int kCarryGroup = 16;  // segment summaries a carry kernel reads before folding them
constexpr int kThreads = 256;  // threads per workgroup of the simple (non-scan) kernels
inline int chunk_steps(int) { return kCK; }
inline int padded_n(int64_t n) { return n <= 8 ? 8 : n <= 16 ? 16 : n <= 32 ? 32 : 64; }
// State padding of the fused kernels: the float-compute kernels use row tiles (at least 16
// states per channel); float64 (dtype code 3) keeps the 8-state minimum.
inline int fused_np(int64_t n, int dtype) {
  const int np = padded_n(n);
  return dtype == 3 || np >= 16 ? np : 16;
}
// LDS rows read with 16-byte vector loads by lanes of different rows are padded by 16 bytes,
// which spreads the lanes of a read over distinct banks.
__host__ __device__ constexpr int ck_pad(int s) { return kCK + 16 / s; }
__host__ __device__ constexpr int np_pad(int s, int np) { return np + 16 / s; }
// gfx950 LDS (measured): a wavefront's 32-bit accesses go in 32-lane halves over 32 banks; its
// 16-byte reads go in 16-lane phases over 64 banks, a phase being lanes {0-3, 12-15, 20-23,
// 24-27} or {4-11, 16-19, 28-31} of a half (the same 32 higher).  When the two channels of a
// half-wavefront each read 16 step rows of np_pad floats at a channel-block stride of 16 rows +
// 16 floats, a phase reads steps {0-3, 12-15} of one channel and {4-11} of the other; this row
// order puts those 16 rows on 16 distinct 16-byte bank groups (the natural order puts 4 pairs on
// one group: 4 extra cycles per read).  Row of step t among a chunk's 16 step rows:
__host__ __device__ constexpr int step_row(int t) { return 4 * (t % 4) + (t < 4 ? 2 : t < 8 ? 0 : t < 12 ? 1 : 3); }
// Channel tile of a fused-kernel workgroup.  MI355X hands workgroup l (linear id x + y *
// gridDim.x) to XCD l % 8, each XCD with its own L2.  Tiles next to each other share 128-byte
// lines of (B, L, D) rows (a 16-channel float32 tile reads 64 bytes of a row per step), so with
// tile = blockIdx.x the two halves of every line went to two XCDs, each fetching the whole
// line.  When gridDim.x is a multiple of 8, XCD k gets tiles [k, k + 1) * gridDim.x / 8 instead.
__device__ __forceinline__ int xcd_tile() {
  const int nx = (int)gridDim.x, x = (int)blockIdx.x;
  return nx % 8 ? x : (x % 8) * (nx / 8) + x / 8;
}
// Low-rank delta (the dt_proj GEMM fused into the staging): a chunk's (CK, R <= kLR) input
// rows and the wavefront's channels' weight rows, padded like the other LDS rows.
constexpr int kLR = 16;
__host__ __device__ constexpr int lr_pad(int s) { return kLR + 16 / s; }
__host__ __device__ constexpr int lr_wave_bytes(int s, int np) { return (kCK + 64 / np) * lr_pad(s) * s; }
__host__ __device__ constexpr int fwd_wave_bytes(int s, int np) {
  return ((2 * (64 / np) + 2 * np) * ck_pad(s) + kCK * (64 / np) * np_pad(s, np)) * s + lr_wave_bytes(s, np);
}
__host__ __device__ constexpr int bwd_half() { return 8; }  // reverse steps per LDS reduction round
__host__ __device__ constexpr int bwd_wave_bytes(int s, int np) {
  return ((6 * (64 / np) + 2 * np) * ck_pad(s) + bwd_half() * (64 / np) * 2 * np_pad(s, np) +
          bwd_half() * 64 * 2) * s + lr_wave_bytes(s, np);
}
__host__ __device__ constexpr int bwd_shared_bytes(int s, int np, int wpb) {
  return wpb > 1 ? 2 * wpb * kCK * np * 2 * s : 0;
}
__host__ __device__ constexpr int fwd_waves(int s, int np) {
  return 4 * fwd_wave_bytes(s, np) <= 65536 ? 4 : 2 * fwd_wave_bytes(s, np) <= 65536 ? 2 : 1;
}
// gfx950 gives a workgroup up to 160 KiB of LDS.  The backward uses as many wavefronts per
// workgroup as fit (up to 8): every extra wavefront widens the channel tile over which dB and
// dC are summed in LDS, and so shrinks the partial sums written to HBM by that factor.
constexpr int kLdsBytes = 160 * 1024;
__host__ __device__ constexpr int bwd_fits(int s, int np, int w) {
  return w * bwd_wave_bytes(s, np) + bwd_shared_bytes(s, np, w) <= kLdsBytes;
}
__host__ __device__ constexpr int bwd_waves(int s, int np) {
  return bwd_fits(s, np, 8) ? 8 : bwd_fits(s, np, 4) ? 4 : bwd_fits(s, np, 2) ? 2 : 1;
}
// Wavefronts per workgroup of the float-compute backward (row tiles, NP >= 16): as many as fit
// in the 160 KiB of LDS (8 at 16 states, 4 at 32 and 64).
__host__ __device__ constexpr int bwdw_waves(int np) { return np <= 16 ? 8 : 4; }
// Channels per backward workgroup (= the channel tile of the dB / dC partial sums).
inline int bwd_channels_per_block(int dtype, int np) {
  if (dtype == 3) return bwd_waves(8, np) * (64 / np);
  return bwdw_waves(np) * (64 / np);
}

struct FwdParams {
  int64_t B, L, D, N;
  int nchunks;
  int softplus;
  int has_D, has_z, has_bias, has_h0, has_last, write_out;
  int uniform;  // all (B,L,D) views share x's strides, C shares B's, row offsets fit in int32
  // Time segments: grid row blockIdx.y = b * nseg + segment; a segment spans seg_chunks chunks.
  // With nseg > 1 a summary pass writes each segment's decay product and zero-start end state
  // (seg_P, seg_E), a carry pass turns them into the state entering each segment (seg_hin),
  // and the main pass starts every segment from seg_hin.  All three are (B, nseg, D, NP).  With
  // at most kFoldSegs segments the float kernels' main pass folds seg_P / seg_E itself and no
  // carry pass runs.
  int nseg, seg_chunks;
  // Chunk pairs between workgroup barriers in the float main pass (0: none).  A (B, L, D)
  // output row takes 16 bytes per step from each of a workgroup's wavefronts; over long
  // segments the wavefronts drift apart and the 64-byte pieces leave L2 before all four parts
  // are written.  The barriers keep them in step.
  int sync_pairs;
  void *seg_P, *seg_E, *seg_hin;
  KView x, dt, A, Bm, Cm, Dsk, z, bias, h0, out, last;
  // Low-rank delta: lowrank = R > 0 means delta = dtl (B, L, R) @ dtw (D, R)^T; dt then
  // aliases x (never read in the uniform layout) so that every tile load stays in bounds.
  int lowrank;
  KView dtl, dtw;
  int a_log;   // A holds A_log: the kernel uses -exp(A_log)
  void *ckpt;  // (B, nchunks, D, NP) state type: state at the end of each chunk
  void *ypre;  // y + D x before the gate (iff gate and saving), state type; the float kernels
               // lay it out (B, D, L), the float64 ones (B, L, D) when x is D-contiguous, else
               // (B, D, L) -- see ypre_index()
};

// Index of (b, t, d) in the saved pre-gate output.  The float kernels always use (B, D, L)
// (dfast = false): a wavefront's 16 steps x 4 channels are then four 64-byte pieces, where
// (B, L, D) gives sixteen 16-byte ones.  The float64 kernels follow x's unit-stride axis.
__host__ __device__ inline int64_t ypre_index(bool dfast, int64_t b, int64_t t, int64_t d, int64_t L, int64_t D) {
  return dfast ? (b * L + t) * D + d : (b * D + d) * L + t;
}

struct BwdParams {
  int64_t B, L, D, N;
  int nchunks, ntiles;
  // Time segments (float kernels): grid row blockIdx.y = b * nseg + segment.  With nseg > 1 a
  // summary pass writes each segment's (E, P) = (first-step decay times its zero-start adjoint,
  // product of its decays), k_bwd_carry turns them into the adjoint entering each segment
  // (seg_mu), and every partial over time (dA, dD, d_bias) gets one row per (b, segment).
  int nseg, seg_chunks;
  void *seg_mu, *seg_E;  // (B, nseg, D, NP) float64
  void *seg_P;           // (B, nseg, D, NP) float32
  int softplus;
  int has_D, has_z, has_bias, has_h0, has_dlast, has_dh0;
  int uniform;  // as in FwdParams
  KView x, dt, A, Bm, Cm, Dsk, z, bias, h0, dout, dlast, dx, ddt, dz, dh0;
  int lowrank;  // as in FwdParams
  KView dtl, dtw;
  int a_log;    // as in FwdParams
  const void *ckpt;
  const void *ypre;
  void *ws_dB, *ws_dC;  // (B, ntiles, L, NP) partial sums over the tile's channels
  void *ws_dA;          // (B, nseg, D, NP) float64 partials over time
  void *ws_dD, *ws_db;  // (B, nseg, D)
};

struct FinParams {
  int64_t B, L, D, N;
  int64_t rows;  // partial rows of dA / dD / d_bias: B * nseg
  int ntiles, np;
  int has_D, has_bias;
  int a_log;  // A holds A_log: dA is written as the gradient of A_log, dA * A
  const void *ws_dB, *ws_dC, *ws_dA, *ws_dD, *ws_db;
  KView A, dB, dC, dA, dD, dbias;
};

struct StepParams {
  int64_t B, D, N;
  int softplus;
  int has_D, has_z, has_bias;
  KView x, dt, A, Bm, Cm, Dsk, z, bias, h, out;
};

// Linear scan h_t = mult_t h_{t-1} + b_t over (B, L, M), processed in the order t = 0..L-1
// (reverse: L-1..0).  shift: mult at a processing position is the a of the previous position
// (1 at the first), which turns the scan into the adjoint recurrence.
struct LscanParams {
  int64_t B, L, M;
  int64_t nc;   // chunks (chunked algorithm)
  int chunk;    // steps per chunk
  int reverse, shift;
  KView a, b, h0, h;  // h0: (B, M) with strides s0, s1
  void *ws;           // chunked: 3 x (B, nc, M) state type (P, E, h_in)
};

// da_t = lambda_t h_prev(t) and dh0 = a_first lambda_first; `reverse` is the forward's direction.
struct LscanGradParams {
  int64_t B, L, M;
  int reverse;
  KView a, h0, h, db, da, dh0;  // db holds lambda
};

// Materialized discretization on contiguous (B, L, D, N) tensors.
struct DiscParams {
  int64_t B, L, D, N;
  int64_t rows_per_group, ngroups, dtiles;
  KView delta, x, A, Bm, ddelta, dx, dA, dBm;
  void *a, *b;
  const void *da, *db;
  void *ws_dB;  // (B*L, dtiles, N) partial sums over each channel tile
  void *ws_dA;  // (ngroups, D, N) partial sums over each group of rows (float64 running sums)
};

// Causal depthwise conv over (B, L, D) views; a lane owns (b, d, one block of TB steps).
// Causal conv: a workgroup covers kConvDG channels x kConvTG lanes of kConvTT time steps
// (kConvTT >= W - 1 for every width <= 8).
constexpr int kConvTT = 8, kConvTG = 4, kConvDG = 64;
struct ConvParams {
  int64_t B, L, D, W;
  int nblk, TB;  // time blocks of kConvTG * kConvTT steps (one workgroup row each), kConvTT
  int silu, has_bias, has_sin, has_sout, has_dbias;
  KView x, w, bias, sin, out, sout, dout, dx, dw, dbias;  // sin / sout: (B, D, W-1)
  void *ws;  // backward: (B * nblk, D, W + 1) partial dweight / dbias, one row per workgroup
};

// RMSNorm over rows of C <= kNormMaxC elements (unit column stride): a wavefront per row,
// kNormWaves wavefronts per workgroup; the backward's wavefronts take norm_rows_per_wave rows.
constexpr int kNormWaves = 4, kNormThreads = kNormWaves * 64, kNormFinThreads = 1024, kNormMaxC = 1024;
// columns per lane (power of two) for a row of C elements
inline constexpr int norm_kc_of(int64_t C) {
  return C <= 64 ? 1 : C <= 128 ? 2 : C <= 256 ? 4 : C <= 512 ? 8 : C <= 1024 ? 16 : 0;
}
inline constexpr int norm_rows_per_wave(int kc) { return kc <= 4 ? 8 : kc == 8 ? 4 : 2; }
struct NormParams {
  int64_t R, C;
  double eps;
  int64_t sx, sy, sdy, sdx;  // row strides (elements)
  const void *x, *w, *dy;
  void *y, *rstd, *dx, *dw;
  void *ws;      // backward: (nblk, C) per-workgroup weight-gradient partials
  int64_t nblk;  // backward workgroups
  int rpw;       // backward rows per wavefront
};

// Fused decode layer (float32, row-major); one workgroup per batch row.
struct DecodeParams {
  int64_t B, dim, N, W, R, dm, P;  // P = R + 2 N
  float eps;
  const float *u, *xz, *conv_w, *conv_b, *x_proj_wt, *dt_proj_w, *dt_bias, *A_log, *Dskip;
  void *conv_state;  // float32, or bf16 when conv_bf16
  int conv_bf16;
  float *ssm_state, *y;
};

// The decode step of a whole layer stack in two launches per layer (ssm_decode_stack).
constexpr int kStThreads = 256;             // threads per workgroup of the stack kernels
constexpr int kInRows = 4, kInCh = 32;      // k_dec_in tile: rows x channels (x and z columns)
constexpr int kScRows = 2, kScCh = 64;      // k_dec_scan tile: rows x channels
constexpr int kStMaxDm = 512, kStMaxDim = 1024;
constexpr int kStMaxInTiles = kStMaxDim / kInCh;   // x_proj partial sums per row
constexpr int kStMaxScTiles = kStMaxDim / kScCh;   // out_proj partial sums per row
struct DecInParams {
  int B, dm, Dm, P, nrt, nct, ndu, write_u, conv_bf16;
  int V;                  // vocabulary (embedding rows; head columns)
  float eps;
  const int64_t *tokens;  // (B,) or null: the residual stream is the embedding rows of the tokens
  const float *embed;     // (V, dm)
  const float *head_w4;   // (dm / 4, V, 4) head weight (the final norm's weight folded in)
  float *logits;          // (B, V)
  const float *u_src;     // (B, dm) residual stream of the previous layer
  const float *du;        // (B, ndu, dm) its out_proj partial sums (ndu = 0: none)
  float *u_dst;           // (B, dm) the residual stream entering this layer (write_u)
  const float *w_in4;     // (dm / 4, 2 Dm, 4)
  const float *conv_w, *conv_b, *x_proj_wt;
  void *conv_state;
  float *xc, *gate, *part;  // (B, Dm), (B, Dm), (B, nct, P)
  int *bad_token;           // status word: set to 1 when a token id lies outside [0, V)
};
struct DecScanParams {
  int B, dm, Dm, N, R, P, nrt, nct, ndu;
  const float *xc, *gate, *part, *dt_proj_w, *dt_bias, *A_log, *Dskip;
  const float *w_out4;    // (Dm / 4, dm, 4)
  float *ssm_state, *du;  // du: (B, ndu, dm)
};
struct DecOutParams {
  int B, dm, ndu;
  const float *u_src, *du;
  float *u_out;
};
hipError_t launch_dec_in(const DecInParams &p, int W, hipStream_t s);
hipError_t launch_dec_scan(const DecScanParams &p, int method, hipStream_t s);
hipError_t launch_dec_out(const DecOutParams &p, hipStream_t s);
hipError_t launch_dec_head(const DecInParams &p, hipStream_t s);

// Runs the summary and carry passes first when p.nseg > 1.
hipError_t launch_fwd(const FwdParams &p, int dtype, int method, int np, hipStream_t s);
hipError_t launch_bwd(const BwdParams &p, int dtype, int method, int np, hipStream_t s);
hipError_t launch_bwd_finalize(const FinParams &p, int dtype, hipStream_t s);
hipError_t launch_step(const StepParams &p, int dtype, int method, int np, hipStream_t s);
hipError_t launch_lscan(const LscanParams &p, int algo, int dtype, hipStream_t s);
hipError_t launch_lscan_grad(const LscanGradParams &p, int dtype, hipStream_t s);
// Channels per workgroup of the discretize backward (its dB partial-sum tile).
inline int disc_channels(int np) { return kThreads / np; }
hipError_t launch_conv(const ConvParams &p, int dtype, bool bwd, hipStream_t s);
hipError_t launch_norm(const NormParams &p, int dtype, bool bwd, hipStream_t s);
size_t decode_shared_bytes(const DecodeParams &p);
hipError_t launch_decode(const DecodeParams &p, int method, hipStream_t s);
hipError_t launch_disc_fwd(const DiscParams &p, int dtype, int method, int np, hipStream_t s);
hipError_t launch_disc_bwd(const DiscParams &p, int dtype, int method, int np, hipStream_t s);

}  // namespace ssm
