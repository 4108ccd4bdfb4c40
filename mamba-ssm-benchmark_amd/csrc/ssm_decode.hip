// Fused scan-path part of a Mamba layer's recurrent decode step for gfx950 (one launch per
// layer): RMSNorm scale, conv step + SiLU with the conv shift state, x_proj, dt_proj + bias +
// softplus, the selective-scan state update, D skip and SiLU(z) gate.  Replaces the ~15 small
// launches of the decode path of models/mamba.py:93-124 (plus the block's RMSNorm) between the
// two GEMMs the caller keeps: in_proj (with the RMSNorm weight folded into its columns) and
// out_proj + residual.
//
// One workgroup of 1024 threads per batch row.  The row's normalized conv output and the x_proj
// results (dt, B, C) live in LDS; x_proj reads its weight channel-major (coalesced across
// outputs) into per-group partial sums that are added in a fixed order.
#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"
#include "ssm_wave.hpp"

namespace ssm {

// The conv state is float32, or bf16 (the state of a bf16-autocast model, models/mamba.py:86-91):
// element j of the state at `base` read as float / written rounded to the state's type.
__device__ __forceinline__ float cs_load(const DecodeParams &p, int64_t i) {
  return p.conv_bf16 ? Conv<bf16_t>::load((const bf16_t *)p.conv_state + i) : ((const float *)p.conv_state)[i];
}
__device__ __forceinline__ void cs_store(const DecodeParams &p, int64_t i, float v) {
  if (p.conv_bf16) Conv<bf16_t>::store((bf16_t *)p.conv_state + i, v);
  else ((float *)p.conv_state)[i] = v;
}

constexpr int kDecThreads = 1024;  // 16 wavefronts per row: every phase is short, latency hides
constexpr int kDecGroups = 16;     // channel groups of the x_proj partial sums

template <int W, int NP, int METHOD>
__global__ void __launch_bounds__(kDecThreads) k_decode(const DecodeParams p) {
  extern __shared__ __align__(16) float dsh[];
  float *xs = dsh;                  // (dim) conv output of this row
  float *zs = xs + p.dim;           // (dim) gate input (normalized)
  float *proj = zs + p.dim;         // (P) x_proj output: dt (R), B (N), C (N)
  float *part = proj + p.P;         // (kDecGroups, P) x_proj partial sums
  float *red = part + kDecGroups * p.P;  // (T / 64) partial sums
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
  constexpr int NW = kDecThreads / kWave;
  const int64_t b = blockIdx.x;
  const int Dm = (int)p.dim, N = (int)p.N, R = (int)p.R, dm = (int)p.dm, P = (int)p.P;

  // RMSNorm scale of the block input (its weight is folded into in_proj by the caller)
  float ss = 0.f;
  for (int k = tid; k < dm; k += kDecThreads) {
    const float v = p.u[b * dm + k];
    ss = fmaf(v, v, ss);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) tot += red[w];
  const float s = rsqrtf(tot / (float)dm + p.eps);

  // conv step + SiLU (models/mamba.py:104-107); the state holds the previous W-1 inputs
  for (int d = tid; d < Dm; d += kDecThreads) {
    const float x = s * p.xz[b * 2 * Dm + d];
    zs[d] = s * p.xz[b * 2 * Dm + Dm + d];
    const int64_t st = (b * Dm + d) * (W - 1);
    float cw[W], win[W > 1 ? W - 1 : 1];
#pragma unroll
    for (int j = 0; j < W; ++j) cw[j] = p.conv_w[d * W + j];
#pragma unroll
    for (int j = 0; j < W - 1; ++j) win[j] = cs_load(p, st + j);
    float acc = fmaf(cw[W - 1], x, p.conv_b[d]);
#pragma unroll
    for (int j = 0; j < W - 1; ++j) acc = fmaf(cw[j], win[j], acc);
#pragma unroll
    for (int j = 0; j + 1 < W - 1; ++j) cs_store(p, st + j, win[j + 1]);
    if constexpr (W > 1) cs_store(p, st + W - 2, x);
    xs[d] = acc * sigmoidf(acc);
  }
  __syncthreads();

  // x_proj, from the channel-major weight (dim, P): thread (group g, output j) sums the
  // channels d = g, g + G, ...; consecutive threads read consecutive outputs of one row
  for (int e = tid; e < kDecGroups * P; e += kDecThreads) {
    const int j = e % P, g = e / P;
    float acc = 0.f;
#pragma unroll 8
    for (int d = g; d < Dm; d += kDecGroups) acc = fmaf(p.x_proj_wt[(int64_t)d * P + j], xs[d], acc);
    part[g * P + j] = acc;
  }
  __syncthreads();
  for (int j = tid; j < P; j += kDecThreads) {
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < kDecGroups; ++g) acc += part[g * P + j];
    proj[j] = acc;
  }
  __syncthreads();

  // dt_proj + bias + softplus, state update, skip and gate: two lanes per channel, each with
  // half of the states; the halves' C h sums meet through one cross-lane add
  constexpr int HN = NP / 2;
  const float *Bv = proj + R, *Cv = proj + R + N;
  for (int e = tid; e < 2 * Dm; e += kDecThreads) {
    const int d = e >> 1, half = e & 1;
    const float *wd = p.dt_proj_w + (int64_t)d * R;
    float dt = p.dt_bias[d];
#pragma unroll 16
    for (int r = 0; r < R; ++r) dt = fmaf(wd[r], proj[r], dt);
    dt = softplusf(dt);
    const float xc = xs[d];
    const int n0 = half * HN;
    float *h = p.ssm_state + (b * Dm + d) * N;
    const float *al = p.A_log + (int64_t)d * N;
    float hr[HN], lr[HN];
#pragma unroll
    for (int i = 0; i < HN; ++i) {
      const int n = n0 + i < N ? n0 + i : N - 1;  // lanes past N read the last state, unused
      hr[i] = h[n];
      lr[i] = al[n];
    }
    float y = 0.f;
#pragma unroll
    for (int i = 0; i < HN; ++i) {
      const int n = n0 + i < N ? n0 + i : N - 1;
      const AConst<float> ac = make_aconst(-__expf(lr[i]));
      float a, coef, hv = hr[i];
      const float bx = Bv[n] * xc;
      if constexpr (METHOD == 0) {
        disc_zoh_m1(dt, ac, a, coef);  // a holds a - 1
        hv = fmaf(a, hv, fmaf(coef, bx, hv));
      } else {
        disc<METHOD>(dt, ac, a, coef);
        hv = fmaf(a, hv, bcoef<METHOD>(dt, coef) * bx);
      }
      hr[i] = hv;
      if (n0 + i < N) y = fmaf(Cv[n], hv, y);
    }
#pragma unroll
    for (int i = 0; i < HN; ++i)
      if (n0 + i < N) h[n0 + i] = hr[i];
    y += __shfl_xor(y, 1);
    if (half == 0) {
      const float zv = zs[d];
      p.y[b * Dm + d] = fmaf(p.Dskip[d], xc, y) * (zv * sigmoidf(zv));
    }
  }
}

// Row-resident variant for the Mamba LM shapes: dim <= 512, dstate 8 or 16, dt_rank 8, 16 or
// 32, d_model <= 1024, conv width <= 4.  Every global read of the row is issued at entry,
// unconditionally and in the order of use (raw buffer reads: past an array's end they return
// 0), so the row costs one memory round trip; the phases after it meet only at LDS barriers and
// every global store comes last.  Thread roles: norm element tid; conv channel tid; x_proj
// wavefront g = channels g, g + 16, ..., lane = output; state pair (2 d, 2 d + 1) = channel d's
// two halves of the states and of the dt rank.
constexpr int kRowGroupCh = 32;  // channels per x_proj wavefront (dim <= 16 * 32)

template <int W, int NPH, int RHALF, int METHOD>
__global__ void __launch_bounds__(kDecThreads) k_decode_row(const DecodeParams p) {
  constexpr int NW = kDecThreads / kWave, N = 2 * NPH, R = 2 * RHALF;
  __shared__ float xs[NW * kRowGroupCh];
  __shared__ float part[NW][kWave];
  __shared__ float proj[kWave];
  __shared__ float red[NW];
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
  const int64_t b = blockIdx.x;
  const int Dm = (int)p.dim, dm = (int)p.dm, P = (int)p.P;

  // raw buffer views (32-bit lane offsets, reads past an extent return 0)
  auto view = [](const float *q, int64_t n) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)q, (short)0, (int)(n * 4), kBufferFlags);
  };
  const auto ru = view(p.u + b * dm, dm), rxz = view(p.xz + b * 2 * Dm, 2 * Dm);
  const auto rcw = view(p.conv_w, Dm * W);
  const int csz = p.conv_bf16 ? 2 : 4;  // conv state element bytes
  const auto rcs = __builtin_amdgcn_make_buffer_rsrc((char *)p.conv_state + b * Dm * (W - 1) * csz, (short)0,
                                                     (int)(Dm * (W - 1) * csz), kBufferFlags);
  const auto rcb = view(p.conv_b, Dm), rxp = view(p.x_proj_wt, (int64_t)Dm * P);
  const auto rdt = view(p.dt_proj_w, (int64_t)Dm * R), rdb = view(p.dt_bias, Dm), rds = view(p.Dskip, Dm);
  const auto rh = view(p.ssm_state + b * Dm * N, Dm * N), ral = view(p.A_log, Dm * N);
  auto ld = [](__amdgpu_buffer_rsrc_t r, int idx) { return buf_load<float>(r, (uint32_t)idx * 4u); };

  const float uv = ld(ru, tid);  // 0 past d_model
  const float xin = ld(rxz, tid);
  float cw[W], st[W > 1 ? W - 1 : 1];
#pragma unroll
  for (int j = 0; j < W; ++j) cw[j] = ld(rcw, tid * W + j);
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const uint32_t o = (uint32_t)(tid * (W - 1) + j);
    st[j] = p.conv_bf16 ? buf_load<bf16_t>(rcs, o * 2u) : buf_load<float>(rcs, o * 4u);
  }
  const float cb = ld(rcb, tid);

  // x_proj weight rows g + 16 k (rows past dim read 0; lanes past P read unused values)
  const int g = __builtin_amdgcn_readfirstlane(wv);
  float wx[kRowGroupCh];
#pragma unroll
  for (int k = 0; k < kRowGroupCh; ++k) wx[k] = ld(rxp, (g + NW * k) * P + lane);

  const int ds = tid >> 1, half = tid & 1, n0 = half * NPH, r0 = half * RHALF;
  float wdt[RHALF];
#pragma unroll
  for (int i = 0; i < RHALF; ++i) wdt[i] = ld(rdt, ds * R + r0 + i);
  const float dtb = ld(rdb, ds), dsk = ld(rds, ds), zin = ld(rxz, Dm + ds);
  float hr[NPH], lr[NPH];
#pragma unroll
  for (int i = 0; i < NPH; ++i) hr[i] = ld(rh, ds * N + n0 + i);
#pragma unroll
  for (int i = 0; i < NPH; ++i) lr[i] = ld(ral, ds * N + n0 + i);

  // RMSNorm scale of the block input (its weight is folded into in_proj by the caller)
  float ss = uv * uv;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) tot += red[w];
  const float s = rsqrtf(tot / (float)dm + p.eps);

  // conv step + SiLU (models/mamba.py:104-107); channels past dim hold 0 for x_proj
  const float x = s * xin;
  float acc = fmaf(cw[W - 1], x, cb);
#pragma unroll
  for (int j = 0; j < W - 1; ++j) acc = fmaf(cw[j], st[j], acc);
  if (tid < NW * kRowGroupCh) xs[tid] = tid < Dm ? acc * sigmoidf(acc) : 0.f;
  __syncthreads();

  // x_proj partial sums per channel group, then the groups in a fixed order
  float pa = 0.f;
#pragma unroll
  for (int k = 0; k < kRowGroupCh; ++k) pa = fmaf(wx[k], xs[g + NW * k], pa);
  part[wv][lane] = pa;
  __syncthreads();
  if (tid < kWave) {
    float a = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) a += part[q][tid];
    proj[tid] = a;
  }
  __syncthreads();

  // dt_proj (each lane of the pair takes half of the rank) + bias + softplus
  float dp = 0.f;
#pragma unroll
  for (int i = 0; i < RHALF; ++i) dp = fmaf(wdt[i], proj[r0 + i], dp);
  const float dt = softplusf(dtb + (dp + __shfl_xor(dp, 1)));

  // state update, C h, skip and gate
  const float xc = xs[min(ds, Dm - 1)];
  const float *Bv = proj + R + n0, *Cv = proj + R + N + n0;
  float y = 0.f;
#pragma unroll
  for (int i = 0; i < NPH; ++i) {
    AConst<float> ac;
    ac.A = -__expf(lr[i]);
    ac.A2 = ac.A * 1.4426950408889634f;
    ac.invA = fast_rcp(ac.A);
    float a, coef, hv = hr[i];
    const float bx = Bv[i] * xc;
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

  if (ds < Dm) {
    float *h = p.ssm_state + (b * Dm + ds) * N + n0;
#pragma unroll
    for (int i = 0; i < NPH; ++i) h[i] = hr[i];
    if (half == 0) {
      const float zv = s * zin;
      p.y[b * Dm + ds] = fmaf(dsk, xc, y) * (zv * sigmoidf(zv));
    }
  }
  if (tid < Dm) {
    const int64_t cst = (b * Dm + tid) * (W - 1);
#pragma unroll
    for (int j = 0; j + 1 < W - 1; ++j) cs_store(p, cst + j, st[j + 1]);
    if constexpr (W > 1) cs_store(p, cst + W - 2, x);
  }
}

bool decode_row_fits(const DecodeParams &p) {
  return p.dim <= kDecThreads / 2 && p.dim <= (int64_t)(kDecThreads / kWave) * kRowGroupCh &&
         (p.N == 8 || p.N == 16) && (p.R == 8 || p.R == 16 || p.R == 32) && p.P <= kWave &&
         p.dm <= kDecThreads && p.W <= 4;
}

template <int W, int NPH, int RHALF>
static void launch_row(const DecodeParams &p, int method, hipStream_t s) {
  const dim3 grid((unsigned)p.B), block(kDecThreads);
  switch (method) {
    case 0: hipLaunchKernelGGL((k_decode_row<W, NPH, RHALF, 0>), grid, block, 0, s, p); break;
    case 1: hipLaunchKernelGGL((k_decode_row<W, NPH, RHALF, 1>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((k_decode_row<W, NPH, RHALF, 2>), grid, block, 0, s, p); break;
  }
}

template <int W, int NP>
static hipError_t decode_m(const DecodeParams &p, int method, size_t shmem, hipStream_t s) {
  const dim3 grid((unsigned)p.B), block(kDecThreads);
  if constexpr (NP <= 16 && W <= 4) {
    if (decode_row_fits(p) && p.N == NP) {
      if (p.R == 8) launch_row<W, NP / 2, 4>(p, method, s);
      else if (p.R == 16) launch_row<W, NP / 2, 8>(p, method, s);
      else launch_row<W, NP / 2, 16>(p, method, s);
      return hipGetLastError();
    }
  }
  switch (method) {
    case 0: hipLaunchKernelGGL((k_decode<W, NP, 0>), grid, block, shmem, s, p); break;
    case 1: hipLaunchKernelGGL((k_decode<W, NP, 1>), grid, block, shmem, s, p); break;
    default: hipLaunchKernelGGL((k_decode<W, NP, 2>), grid, block, shmem, s, p); break;
  }
  return hipGetLastError();
}

template <int W>
static hipError_t decode_n(const DecodeParams &p, int method, size_t shmem, hipStream_t s) {
  switch (padded_n(p.N)) {
    case 8: return decode_m<W, 8>(p, method, shmem, s);
    case 16: return decode_m<W, 16>(p, method, shmem, s);
    case 32: return decode_m<W, 32>(p, method, shmem, s);
    default: return decode_m<W, 64>(p, method, shmem, s);
  }
}

size_t decode_shared_bytes(const DecodeParams &p) {
  return (size_t)(2 * p.dim + (1 + kDecGroups) * p.P + kDecThreads / kWave) * sizeof(float);
}

hipError_t launch_decode(const DecodeParams &p, int method, hipStream_t s) {
  const size_t shmem = decode_shared_bytes(p);
  switch (p.W) {
    case 1: return decode_n<1>(p, method, shmem, s);
    case 2: return decode_n<2>(p, method, shmem, s);
    case 3: return decode_n<3>(p, method, shmem, s);
    case 4: return decode_n<4>(p, method, shmem, s);
    case 5: return decode_n<5>(p, method, shmem, s);
    case 6: return decode_n<6>(p, method, shmem, s);
    case 7: return decode_n<7>(p, method, shmem, s);
    default: return decode_n<8>(p, method, shmem, s);
  }
}

}  // namespace ssm
