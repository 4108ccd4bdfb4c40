// The recurrent decode step of a stack of Mamba layers -- the residual stream through every
// block (models/lm.py:124-128 with states; per block models/lm.py:82-83 with the RMSNorm of
// models/common.py:14-16 and the mixer of models/mamba.py:93-124 at L = 1) -- in two launches
// per layer, each spread over the whole GPU instead of one workgroup per batch row:
//
//   k_dec_in    workgroup = 4 batch rows x 32 channels: the residual stream rebuilt from the
//               previous layer's out_proj partial sums, the RMSNorm scale of its rows, the
//               tile of the in_proj GEMM (x and z columns; the norm weight folded into the
//               weight), the conv step + SiLU with the conv state, the SiLU(z) gate, and the
//               x_proj partial sums over the tile's channels;
//   k_dec_scan  workgroup = 2 batch rows x 64 channels: the x_proj sums finished, dt_proj +
//               bias + softplus, the state update, C h, D skip and gate, and the out_proj
//               partial sums over the tile's channels.
//
// The token step's ends fold into the same kernels: block 0's k_dec_in may read the embedding
// rows of the tokens as its residual stream (models/lm.py:125), and k_dec_in with its head
// epilogue (HEAD: the rebuild, RMSNorm scale and GEMM over vocabulary columns) gives the logits
// of the final norm and the head (models/lm.py:128); without a head, k_dec_out adds the last
// layer's partial sums to its residual stream.  Every reduction runs in a fixed order, so the
// step is deterministic.  A workgroup issues its global reads (states, weights, partial sums)
// at entry, so each launch costs one memory round trip; workgroups are grouped on XCDs
// (blockIdx mod 8) by the weight tiles and rows they share, so each is read into few L2s.
#include "ssm_device.hpp"
#include "ssm_dpp.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"
#include "ssm_wave.hpp"

namespace ssm {

// blockIdx -> linear tile id, the workgroups of one XCD (blockIdx mod 8) on consecutive ids:
// a bijection of [0, g).
__device__ __forceinline__ int xcd_linear(int i, int g) {
  const int x = i & 7, s = i >> 3, q = g >> 3, rem = g & 7;
  return x * q + min(x, rem) + s;
}

// Element idx of a float buffer (0 past its extent).
__device__ __forceinline__ float ldf(__amdgpu_buffer_rsrc_t r, int idx) { return buf_load<float>(r, (uint32_t)idx * 4u); }
__device__ __forceinline__ void stf(__amdgpu_buffer_rsrc_t r, int idx, bool ok, float v) {
  buf_store<float>(r, (uint32_t)idx * 4u, ok, v);
}
// Elements idx .. idx + 3 (idx a multiple of 4 from a 16-byte aligned base; 0 past the extent).
__device__ __forceinline__ float4 ldf4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}
__device__ __forceinline__ void stf4(__amdgpu_buffer_rsrc_t r, uint32_t off, bool ok, float4 v) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const u4 q = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
  __builtin_amdgcn_raw_buffer_store_b128(q, r, (int)(ok ? off : kDropOffset), 0, 0);
}
__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

constexpr int kInKB = 64;  // in_proj k values per wavefront per pass (4 wavefronts: 256 per pass)

// Sum over the wavefront, every lane receiving the same bits (fixed order).
__device__ __forceinline__ float wave_sum(float v) {
  const float r = row_sum(v);
  auto lane_val = [](float x, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
  };
  return (lane_val(r, 0) + lane_val(r, 16)) + (lane_val(r, 32) + lane_val(r, 48));
}

// KQ passes of 256 over d_model; NDU >= the previous block's partial sums per row (0: none).
// Roles: rebuild and RMSNorm = row wv (lane: elements 4 lane .. 4 lane + 3 of each pass);
// epilogue = row wv, column lane (x channel c0 + lane for lane < 32, else z channel
// c0 + lane - 32); in_proj = the wavefront's quarter of k for the 4 rows on the matrix cores,
// lane's column; x_proj = row wv, output lane.  HEAD: the columns are the 64 vocabulary entries
// of tile ct and the epilogue stores the logits.
template <int W, int KQ, int NDU, bool HEAD>
__global__ void __launch_bounds__(kStThreads) k_dec_in(const DecInParams p) {
  constexpr int NWV = kStThreads / kWave;
  constexpr int KP = KQ * NWV * kInKB;        // padded d_model
  constexpr int XPN = kInCh * kWave / kStThreads;  // x_proj weight reads per thread
  static_assert(NWV == kInRows && 2 * kInCh == kWave, "one epilogue row per wavefront");
  __shared__ __align__(16) float us[kInRows][KP];
  __shared__ float gsum[NWV][kInRows][kWave];
  __shared__ float xcs[kInRows][kInCh];
  __shared__ float xps[kInCh * kWave];        // x_proj weight rows of the tile, (kInCh, P) row-major
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid >> 6;
  // XCD grouping: where the grid allows, XCD x takes row half x / 4 and column quarter x % 4,
  // so each XCD's L2 holds a quarter of the weight tiles and half of the partial-sum rows;
  // otherwise the workgroups sharing a weight tile run on one XCD
  int ct, rt;
  if (p.nrt % 2 == 0 && p.nct % 4 == 0 && gridDim.x % 8 == 0) {
    const int x = blockIdx.x & 7, s = blockIdx.x >> 3, hr = p.nrt / 2;
    rt = (x >> 2) * hr + s % hr;
    ct = (x & 3) * (p.nct / 4) + s / hr;
  } else {
    const int L = xcd_linear(blockIdx.x, gridDim.x);
    ct = L / p.nrt;
    rt = L - ct * p.nrt;
  }
  const int b0 = rt * kInRows, c0 = ct * kInCh;
  const int B = p.B, dm = p.dm, Dm = p.Dm, P = p.P, ndu = p.ndu;

  // every global read first, in the order of first use: the residual stream (or the token's
  // embedding row: an id outside the vocabulary reads a zero row) and the partial sums
  const bool emb = p.tokens != nullptr;
  const auto ru = emb ? flat_buffer(p.embed, (int64_t)p.V * dm * 4) : flat_buffer(p.u_src, (int64_t)B * dm * 4);
  const auto rdu = flat_buffer(p.du, (int64_t)B * ndu * dm * 4);
  // rebuild role: row wv, elements k4 .. k4 + 3, k4 = 4 lane + 256 q (d_model a multiple of 4)
  float4 uv[KQ], dv[KQ][NDU > 0 ? NDU : 1];
  {
    const int b = b0 + wv;  // rows past the batch read 0
    int64_t row = b;
    if (emb) row = b < B ? p.tokens[b] : -1;
    const bool rok = row >= 0 && row < (emb ? p.V : B);
    // an id outside the vocabulary reads a zero row and raises the call's status word (a vector
    // store from one lane of the row's wavefront; every workgroup of the row stores the same 1)
    if (emb && b < B && !rok && lane == 0) *(volatile int *)p.bad_token = 1;
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
      const int k4 = 4 * lane + q * kStThreads;
      uv[q] = ldf4(ru, rok ? (uint32_t)(row * dm + k4) * 4u : kDropOffset);
#pragma unroll
      for (int t = 0; t < NDU; ++t) dv[q][t] = ldf4(rdu, t < ndu ? (uint32_t)((b * ndu + t) * dm + k4) * 4u : kDropOffset);
    }
  }

  const int r = wv, j = lane, d = c0 + (j & (kInCh - 1)), b = b0 + r;
  const bool ok = b < B && d < Dm;
  const int bc = min(b, B - 1), dc = min(d, Dm - 1);
  const auto rcw = flat_buffer(p.conv_w, (int64_t)Dm * W * 4), rcb = flat_buffer(p.conv_b, (int64_t)Dm * 4);
  const int csz = p.conv_bf16 ? 2 : 4;
  const auto rcs = flat_buffer(p.conv_state, (int64_t)B * Dm * (W - 1) * csz);
  const int cst = (bc * Dm + dc) * (W - 1);
  float cw[W], st[W > 1 ? W - 1 : 1];
#pragma unroll
  for (int i = 0; i < W; ++i) cw[i] = HEAD ? 0.f : ldf(rcw, dc * W + i);
#pragma unroll
  for (int i = 0; i < W - 1; ++i)
    st[i] = p.conv_bf16 ? buf_load<bf16_t>(rcs, (uint32_t)(cst + i) * 2u) : ldf(rcs, cst + i);
  const float cb = HEAD ? 0.f : ldf(rcb, dc);
  const auto rxp = flat_buffer(p.x_proj_wt, (int64_t)Dm * P * 4);
  float xpv[XPN];
#pragma unroll
  for (int i = 0; i < XPN; ++i) xpv[i] = HEAD ? 0.f : ldf(rxp, c0 * P + tid + i * kStThreads);  // 0 past dim

  // GEMM weight column of this lane, four k per read from the (d_model / 4, ncol, 4) layout (a
  // channel or vocabulary entry past the end reads a valid column whose results are never
  // used), k split over the wavefronts
  const int ncol = HEAD ? p.V : 2 * Dm;
  const auto rw = flat_buffer(HEAD ? p.head_w4 : p.w_in4, (int64_t)dm * ncol * 4);
  const int col = HEAD ? min(ct * kWave + lane, p.V - 1) : (lane < kInCh ? 0 : Dm) + min(c0 + (lane & (kInCh - 1)), Dm - 1);
  float4 wr[KQ][kInKB / 4];
#pragma unroll
  for (int q = 0; q < KQ; ++q)
#pragma unroll
    for (int i = 0; i < kInKB / 4; ++i)  // 0 past d_model
      wr[q][i] = ldf4(rw, (uint32_t)(((q * NWV + wv) * (kInKB / 4) + i) * ncol + col) * 16u);

  // residual stream of row wv: u + the previous block's partial sums in order
#pragma unroll
  for (int q = 0; q < KQ; ++q) {
    const int k4 = 4 * lane + q * kStThreads;
    float4 v = uv[q];
#pragma unroll
    for (int t = 0; t < NDU; ++t) v = add4(v, dv[q][t]);
    if (k4 >= dm) v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p.write_u && ct == 0)
      stf4(flat_buffer(p.u_dst, (int64_t)B * dm * 4), (uint32_t)((b0 + wv) * dm + k4) * 4u, b0 + wv < B && k4 < dm, v);
    *(float4 *)&us[wv][k4] = v;
  }
#pragma unroll
  for (int i = 0; i < XPN; ++i) {
    const int e = tid + i * kStThreads;
    if (e < kInCh * P) xps[e] = xpv[i];
  }
  __syncthreads();

  // RMSNorm scale of row wv (its weight is folded into in_proj)
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < KP / kWave; ++i) {
    const float v = us[r][lane + i * kWave];
    ss = fmaf(v, v, ss);
  }
  const float s = rsqrtf(wave_sum(ss) / (float)dm + p.eps);

  // in_proj on the matrix cores, this wavefront's quarter of k for the 4 rows:
  // v_mfma_f32_4x4x1f32 computes 16 blocks of (4 rows x 1 k) x (1 k x 4 columns); lane l gives
  // row l % 4's stream value and the weight of its own column l, and receives the 4 rows' sums
  // of column l.  Four accumulators (k mod 4) keep four independent chains in flight; they and
  // then the wavefronts' quarters are added in a fixed order.
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 cacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) cacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int ur = lane & (kInRows - 1);
#pragma unroll
  for (int q = 0; q < KQ; ++q) {
    const int kb = (q * NWV + wv) * kInKB;
#pragma unroll
    for (int i = 0; i < kInKB / 4; ++i) {
      const float4 u4 = *(const float4 *)&us[ur][kb + 4 * i];
      const float4 w = wr[q][i];
      cacc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(u4.x, w.x, cacc[0], 0, 0, 0);
      cacc[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(u4.y, w.y, cacc[1], 0, 0, 0);
      cacc[2] = __builtin_amdgcn_mfma_f32_4x4x1f32(u4.z, w.z, cacc[2], 0, 0, 0);
      cacc[3] = __builtin_amdgcn_mfma_f32_4x4x1f32(u4.w, w.w, cacc[3], 0, 0, 0);
    }
  }
  float acc[kInRows];
#pragma unroll
  for (int rr = 0; rr < kInRows; ++rr) acc[rr] = (cacc[0][rr] + cacc[1][rr]) + (cacc[2][rr] + cacc[3][rr]);
#pragma unroll
  for (int rr = 0; rr < kInRows; ++rr) gsum[wv][rr][lane] = acc[rr];
  __syncthreads();
  const float v = s * (((gsum[0][r][j] + gsum[1][r][j]) + gsum[2][r][j]) + gsum[3][r][j]);
  if constexpr (HEAD) {
    const int vc = ct * kWave + lane;
    stf(flat_buffer(p.logits, (int64_t)B * p.V * 4), b * p.V + vc, b < B && vc < p.V, v);
    return;
  }

  // conv step + SiLU (models/mamba.py:104-107) for x columns, the gate SiLU(z) for z columns
  const int io = b * Dm + d;
  if (j < kInCh) {
    float a = fmaf(cw[W - 1], v, cb);
#pragma unroll
    for (int i = 0; i < W - 1; ++i) a = fmaf(cw[i], st[i], a);
    const float xcv = ok ? a * sigmoidf(a) : 0.f;
    xcs[r][j] = xcv;
    stf(flat_buffer(p.xc, (int64_t)B * Dm * 4), io, ok, xcv);
    const int co = io * (W - 1);
    if (p.conv_bf16) {
#pragma unroll
      for (int i = 0; i + 1 < W - 1; ++i) buf_store<bf16_t>(rcs, (uint32_t)(co + i) * 2u, ok, st[i + 1]);
      if constexpr (W > 1) buf_store<bf16_t>(rcs, (uint32_t)(co + W - 2) * 2u, ok, v);
    } else {
#pragma unroll
      for (int i = 0; i + 1 < W - 1; ++i) stf(rcs, co + i, ok, st[i + 1]);
      if constexpr (W > 1) stf(rcs, co + W - 2, ok, v);
    }
  } else {
    stf(flat_buffer(p.gate, (int64_t)B * Dm * 4), io, ok, v * sigmoidf(v));
  }
  __syncthreads();

  // x_proj partial sums over this tile's channels (channels past dim hold 0)
  float pa = 0.f;
#pragma unroll
  for (int i = 0; i < kInCh; ++i) pa = fmaf(xcs[r][i], xps[min(i * P + lane, kInCh * kWave - 1)], pa);
  stf(flat_buffer(p.part, (int64_t)B * p.nct * P * 4), (b * p.nct + ct) * P + lane, b < B && lane < P, pa);
}

// NCT >= the x_proj partial sums per row.  Roles: x_proj sums = row wv (wavefronts 0, 1),
// output lane; state = channel pair (row, d), each of its two lanes half of the states and of the
// dt rank; out_proj = column tid + 256 q.
template <int NPH, int RHALF, int METHOD, int KQ, int NCT>
__global__ void __launch_bounds__(kStThreads) k_dec_scan(const DecScanParams p) {
  constexpr int N = 2 * NPH, R = 2 * RHALF;
  static_assert(2 * kScRows * kScCh == kStThreads, "two lanes per (row, channel)");
  __shared__ float proj[kScRows][kWave];
  __shared__ __align__(16) float ys[kScRows][kScCh];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid >> 6;
  const int L = xcd_linear(blockIdx.x, gridDim.x);
  const int c2 = L / p.nrt, rt = L - c2 * p.nrt;
  const int b0 = rt * kScRows, c0 = c2 * kScCh;
  const int B = p.B, dm = p.dm, Dm = p.Dm, P = p.P, nct = p.nct;

  // every global read first, the states (the longest to arrive) leading
  const int pr = tid >> 1, half = tid & 1, r = pr / kScCh, dl = pr % kScCh;
  const int b = b0 + r, d = c0 + dl;
  const bool ok = b < B && d < Dm;
  const int bc = min(b, B - 1), dc = min(d, Dm - 1), n0 = half * NPH, r0 = half * RHALF;
  const auto rh = flat_buffer(p.ssm_state, (int64_t)B * Dm * N * 4);
  const auto ral = flat_buffer(p.A_log, (int64_t)Dm * N * 4);
  float hr[NPH], lr[NPH];
#pragma unroll
  for (int i = 0; i < NPH; i += 4) {
    const float4 h4 = ldf4(rh, (uint32_t)((bc * Dm + dc) * N + n0 + i) * 4u);
    hr[i] = h4.x; hr[i + 1] = h4.y; hr[i + 2] = h4.z; hr[i + 3] = h4.w;
  }
#pragma unroll
  for (int i = 0; i < NPH; i += 4) {
    const float4 a4 = ldf4(ral, (uint32_t)(dc * N + n0 + i) * 4u);
    lr[i] = a4.x; lr[i + 1] = a4.y; lr[i + 2] = a4.z; lr[i + 3] = a4.w;
  }
  float pv[NCT];
  if (wv < kScRows) {
    const auto rpart = flat_buffer(p.part, (int64_t)B * nct * P * 4);
    const int b = b0 + wv;  // rows past the batch read 0
#pragma unroll
    for (int t = 0; t < NCT; ++t) pv[t] = t < nct ? ldf(rpart, (b * nct + t) * P + lane) : 0.f;
  }
  const auto rdt = flat_buffer(p.dt_proj_w, (int64_t)Dm * R * 4);
  float wdt[RHALF];
#pragma unroll
  for (int i = 0; i < RHALF; i += 4) {
    const float4 w4 = ldf4(rdt, (uint32_t)(dc * R + r0 + i) * 4u);
    wdt[i] = w4.x; wdt[i + 1] = w4.y; wdt[i + 2] = w4.z; wdt[i + 3] = w4.w;
  }
  const float dtb = ldf(flat_buffer(p.dt_bias, (int64_t)Dm * 4), dc);
  const float dsk = ldf(flat_buffer(p.Dskip, (int64_t)Dm * 4), dc);
  const float xcv = ldf(flat_buffer(p.xc, (int64_t)B * Dm * 4), bc * Dm + dc);
  const float gv = ldf(flat_buffer(p.gate, (int64_t)B * Dm * 4), bc * Dm + dc);
  const auto rwo = flat_buffer(p.w_out4, (int64_t)Dm * dm * 4);  // (dim / 4, d_model, 4)
  float4 wo[KQ][kScCh / 4];
#pragma unroll
  for (int q = 0; q < KQ; ++q)
#pragma unroll
    for (int i = 0; i < kScCh / 4; ++i)  // 0 past dim
      wo[q][i] = ldf4(rwo, (uint32_t)((c0 / 4 + i) * dm + tid + q * kStThreads) * 16u);

  // x_proj outputs of the 2 rows: the partial sums in order
  if (wv < kScRows) {
    float a = 0.f;
#pragma unroll
    for (int t = 0; t < NCT; ++t) a += pv[t];
    proj[wv][lane] = a;
  }
  __syncthreads();

  // dt_proj + bias + softplus (models/mamba.py:75-76), the state update, C h, skip and gate
  float dp = 0.f;
#pragma unroll
  for (int i = 0; i < RHALF; ++i) dp = fmaf(wdt[i], proj[r][r0 + i], dp);
  const float dt = softplusf(dtb + (dp + __shfl_xor(dp, 1)));
  const float *Bv = &proj[r][R + n0], *Cv = &proj[r][R + N + n0];
  float y = 0.f;
#pragma unroll
  for (int i = 0; i < NPH; ++i) {
    AConst<float> ac;
    ac.A = -__expf(lr[i]);
    ac.A2 = ac.A * 1.4426950408889634f;
    ac.invA = fast_rcp(ac.A);
    float a, coef, hv = hr[i];
    const float bx = Bv[i] * xcv;
    if constexpr (METHOD == 0) {
      disc_zoh_m1(dt, ac, a, coef);  // a holds a - 1
      hv = fmaf(a, hv, fmaf(coef, bx, hv));
    } else {
      disc<METHOD>(dt, ac, a, coef);
      hv = fmaf(a, hv, bcoef<METHOD>(dt, coef) * bx);
    }
    hr[i] = hv;
    y = fmaf(Cv[i], hv, y);
  }
  y += __shfl_xor(y, 1);
  if (half == 0) ys[r][dl] = ok ? fmaf(dsk, xcv, y) * gv : 0.f;
#pragma unroll
  for (int i = 0; i < NPH; i += 4)
    stf4(rh, (uint32_t)((b * Dm + d) * N + n0 + i) * 4u, ok, make_float4(hr[i], hr[i + 1], hr[i + 2], hr[i + 3]));
  __syncthreads();

  // out_proj partial sums over this tile's channels (channels past dim hold 0)
  const auto rdu = flat_buffer(p.du, (int64_t)B * p.ndu * dm * 4);
#pragma unroll
  for (int q = 0; q < KQ; ++q) {
    const int jo = tid + q * kStThreads;
#pragma unroll
    for (int rr = 0; rr < kScRows; ++rr) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < kScCh; i += 4) {
        const float4 y4 = *(const float4 *)&ys[rr][i], w = wo[q][i / 4];
        a = fmaf(y4.x, w.x, a);
        a = fmaf(y4.y, w.y, a);
        a = fmaf(y4.z, w.z, a);
        a = fmaf(y4.w, w.w, a);
      }
      stf(rdu, ((b0 + rr) * p.ndu + c2) * dm + jo, b0 + rr < B && jo < dm, a);
    }
  }
}

// The residual stream leaving the last layer: its input plus its partial sums in order.
__global__ void __launch_bounds__(kStThreads) k_dec_out(const DecOutParams p) {
  const int i = blockIdx.x * kStThreads + threadIdx.x;
  if (i >= p.B * p.dm) return;
  const int b = i / p.dm, k = i - b * p.dm;
  float v = p.u_src[i];
  for (int t = 0; t < p.ndu; ++t) v += p.du[(b * p.ndu + t) * p.dm + k];
  p.u_out[i] = v;
}

template <int W, int KQ, bool HEAD = false>
static void launch_in_q(const DecInParams &p, dim3 grid, hipStream_t s) {
  if (p.ndu == 0) hipLaunchKernelGGL((k_dec_in<W, KQ, 0, HEAD>), grid, dim3(kStThreads), 0, s, p);
  else if (p.ndu <= kStMaxScTiles / 2)
    hipLaunchKernelGGL((k_dec_in<W, KQ, kStMaxScTiles / 2, HEAD>), grid, dim3(kStThreads), 0, s, p);
  else hipLaunchKernelGGL((k_dec_in<W, KQ, kStMaxScTiles, HEAD>), grid, dim3(kStThreads), 0, s, p);
}

// The final norm and the head: k_dec_in's rebuild, norm scale and GEMM over vocabulary tiles.
hipError_t launch_dec_head(const DecInParams &p, hipStream_t s) {
  const dim3 grid((unsigned)(p.nrt * p.nct));
  if (p.dm > kStThreads) launch_in_q<1, 2, true>(p, grid, s);
  else launch_in_q<1, 1, true>(p, grid, s);
  return hipGetLastError();
}

template <int W>
static void launch_in_w(const DecInParams &p, dim3 grid, hipStream_t s) {
  if (p.dm > kStThreads) launch_in_q<W, 2>(p, grid, s);
  else launch_in_q<W, 1>(p, grid, s);
}

hipError_t launch_dec_in(const DecInParams &p, int W, hipStream_t s) {
  const dim3 grid((unsigned)(p.nrt * p.nct));
  switch (W) {
    case 1: launch_in_w<1>(p, grid, s); break;
    case 2: launch_in_w<2>(p, grid, s); break;
    case 3: launch_in_w<3>(p, grid, s); break;
    default: launch_in_w<4>(p, grid, s); break;
  }
  return hipGetLastError();
}

template <int NPH, int RHALF, int METHOD, int KQ>
static void launch_scan_q(const DecScanParams &p, dim3 grid, hipStream_t s) {
  if (p.nct <= kStMaxInTiles / 2) hipLaunchKernelGGL((k_dec_scan<NPH, RHALF, METHOD, KQ, kStMaxInTiles / 2>), grid, dim3(kStThreads), 0, s, p);
  else hipLaunchKernelGGL((k_dec_scan<NPH, RHALF, METHOD, KQ, kStMaxInTiles>), grid, dim3(kStThreads), 0, s, p);
}

template <int NPH, int RHALF, int METHOD>
static void launch_scan_m(const DecScanParams &p, dim3 grid, hipStream_t s) {
  if (p.dm > kStThreads) launch_scan_q<NPH, RHALF, METHOD, 2>(p, grid, s);
  else launch_scan_q<NPH, RHALF, METHOD, 1>(p, grid, s);
}

template <int NPH, int RHALF>
static void launch_scan_r(const DecScanParams &p, int method, dim3 grid, hipStream_t s) {
  switch (method) {
    case 0: launch_scan_m<NPH, RHALF, 0>(p, grid, s); break;
    case 1: launch_scan_m<NPH, RHALF, 1>(p, grid, s); break;
    default: launch_scan_m<NPH, RHALF, 2>(p, grid, s); break;
  }
}

template <int NPH>
static void launch_scan_n(const DecScanParams &p, int method, dim3 grid, hipStream_t s) {
  switch (p.R) {
    case 8: launch_scan_r<NPH, 4>(p, method, grid, s); break;
    case 16: launch_scan_r<NPH, 8>(p, method, grid, s); break;
    default: launch_scan_r<NPH, 16>(p, method, grid, s); break;
  }
}

hipError_t launch_dec_scan(const DecScanParams &p, int method, hipStream_t s) {
  const dim3 grid((unsigned)(p.nrt * p.ndu));
  if (p.N == 8) launch_scan_n<4>(p, method, grid, s);
  else launch_scan_n<8>(p, method, grid, s);
  return hipGetLastError();
}

hipError_t launch_dec_out(const DecOutParams &p, hipStream_t s) {
  const int n = p.B * p.dm;
  hipLaunchKernelGGL(k_dec_out, dim3((unsigned)((n + kStThreads - 1) / kStThreads)), dim3(kStThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace ssm
