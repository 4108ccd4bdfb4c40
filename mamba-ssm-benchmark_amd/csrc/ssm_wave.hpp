// Wavefront-level geometry and staging for the fused scan kernels.
//
// Every 64-lane wavefront works on its own CW = 64/NP channels: lane (c, n) = (lane / NP,
// lane % NP) owns the state h[c, n].  A wavefront stages what its lanes need into a private
// LDS region and reads it back without any workgroup barrier (a wavefront's LDS operations
// complete in issue order, so only compiler reordering has to be fenced).  Two tile shapes
// are staged per chunk of CK steps:
//   (t, c) tiles -- CK x CW per-channel values (x, delta, z, dy, ...): element e of a tile is
//                   handled by lane e % 64; the element -> (t, c) map walks the tensor's unit
//                   stride axis across consecutive lanes, so global accesses are coalesced for
//                   time-major (B,L,D) and channel-major (B,D,L) storage alike;
//   (t, n) tiles -- CK x NP per-state values (B, C) shared by all channels.
// Rows are stored time-contiguous ([c][t], [n][t]) and padded to 16-byte multiples so a lane
// reads a run of steps with 16-byte LDS loads.
#pragma once

#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"

namespace ssm {

constexpr int kWave = 64;

// Compiler fence for wavefront-private LDS traffic (no hardware barrier is needed).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier ordering LDS traffic only: global loads and stores stay in flight across it
// (a full __syncthreads() would first drain them with vmcnt(0)).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename CT> struct WaveCfg {
  static constexpr int CK = 16;                          // steps per chunk (checkpoint interval)
  static constexpr int CKP = CK + 16 / (int)sizeof(CT);  // padded row length
};

// Element e of a ROWS (time) x COLS tile -> (t, c); tfast = the time axis has unit stride.
template <int ROWS, int COLS>
__device__ __forceinline__ void tc_of(int e, bool tfast, int &t, int &c) {
  if (tfast) {
    t = e % ROWS;
    c = e / ROWS;
  } else {
    t = e / COLS;
    c = e % COLS;
  }
}

// Element offset of (t, c) inside one batch row.  With a uniform layout (UL) every offset of
// the row is known to fit in 32 bits (checked on the host), which keeps the address arithmetic
// in 32-bit VALU ops.
template <bool UL>
__device__ __forceinline__ int64_t row_off(int t, int c, int64_t s1, int64_t s2) {
  if (UL) return (int64_t)(t * (int)s1 + c * (int)s2);
  return (int64_t)t * s1 + (int64_t)c * s2;
}

// With a uniform layout all (B, L, D) tensors share x's strides and C shares B's: kernels read
// the strides from one view so the compiler computes each address once.
template <bool UL>
__device__ __forceinline__ KView with_layout(const KView &v, const KView &ref) {
  return UL ? KView{v.p, ref.s0, ref.s1, ref.s2} : v;
}

// ------------------------------------------------------------------ raw buffer reads
// With a uniform layout every batch row of a view spans less than 2^31 bytes (checked on the
// host), so a tile element is addressed by a 32-bit byte offset from the row's base through a
// buffer resource whose range is the row's extent: the per-lane offsets are computed once per
// kernel, a chunk adds one uniform offset, and a read past the extent returns 0 instead of
// faulting (so no clamping is needed for the ragged last chunk or channel tile).
constexpr int kBufferFlags = 0x00020000;  // raw 32-bit data, gfx9 family

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_buffer(const KView &V, int64_t b, int L, int C, int esize) {
  const char *base = (const char *)V.p + b * V.s0 * esize;
  const int64_t ext = ((int64_t)(L - 1) * V.s1 + (int64_t)(C - 1) * V.s2 + 1) * esize;
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)ext, kBufferFlags);
}

template <typename IT> __device__ __forceinline__ typename Conv<IT>::CT buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ float buf_load<float>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
template <> __device__ __forceinline__ float buf_load<bf16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __uint_as_float(((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0)) << 16);
}
template <> __device__ __forceinline__ float buf_load<f16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (float)__builtin_bit_cast(f16_t, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0));
}
template <> __device__ __forceinline__ double buf_load<double>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}
// The same with a uniform (scalar) offset added by the hardware: a chunk's offset costs no VALU.
// The range check covers the vector offset only, so these serve reads known to lie inside the
// buffer; a read that may run past it puts its whole offset in `off` (buf_load).
template <typename IT> __device__ __forceinline__ float buf_load_s(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff);
template <> __device__ __forceinline__ float buf_load_s<float>(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, (int)soff, 0));
}
template <> __device__ __forceinline__ float buf_load_s<bf16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
  return __uint_as_float(((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, (int)soff, 0)) << 16);
}
template <> __device__ __forceinline__ float buf_load_s<f16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
  return (float)__builtin_bit_cast(f16_t, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, (int)soff, 0));
}

// Raw buffer stores.  A lane whose `ok` is false stores to an offset past the buffer's extent
// (every row buffer the host allows spans less than 2^31 bytes), which the hardware discards:
// a masked store needs no branch, so a chunk's code stays one basic block.
constexpr uint32_t kDropOffset = 0x80000000u;
template <typename IT> __device__ __forceinline__ void buf_store(__amdgpu_buffer_rsrc_t r, uint32_t off, bool ok, float v);
template <> __device__ __forceinline__ void buf_store<float>(__amdgpu_buffer_rsrc_t r, uint32_t off, bool ok, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)(ok ? off : kDropOffset), 0, 0);
}
template <> __device__ __forceinline__ void buf_store<bf16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off, bool ok, float v) {
  bf16_t q;
  Conv<bf16_t>::store(&q, v);
  __builtin_amdgcn_raw_buffer_store_b16(q.bits, r, (int)(ok ? off : kDropOffset), 0, 0);
}
template <> __device__ __forceinline__ void buf_store<f16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off, bool ok, float v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (f16_t)v), r, (int)(ok ? off : kDropOffset), 0, 0);
}
// Masked store with a uniform offset added by the hardware (`ok` false: dropped).
template <typename IT> __device__ __forceinline__ void buf_store_s(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff, bool ok, float v);
template <> __device__ __forceinline__ void buf_store_s<float>(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff, bool ok, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)(ok ? off : kDropOffset), (int)soff, 0);
}
template <> __device__ __forceinline__ void buf_store_s<bf16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff, bool ok, float v) {
  bf16_t q;
  Conv<bf16_t>::store(&q, v);
  __builtin_amdgcn_raw_buffer_store_b16(q.bits, r, (int)(ok ? off : kDropOffset), (int)soff, 0);
}
template <> __device__ __forceinline__ void buf_store_s<f16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff, bool ok, float v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (f16_t)v), r, (int)(ok ? off : kDropOffset), (int)soff, 0);
}
// A buffer over `bytes` bytes at `base` (0 bytes: every access is dropped / reads 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t flat_buffer(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, kBufferFlags);
}

// The kernel's parameter block (its only argument, at the start of the kernarg segment), read
// through a pointer the compiler cannot see through: fields read after a long loop are loaded
// there, instead of being loaded at entry and held (or spilled) across the loop.
template <typename P>
__device__ __forceinline__ const P &params_here() {
  const __attribute__((address_space(4))) P *pk =
      (const __attribute__((address_space(4))) P *)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(pk));
  return *(const P *)pk;  // the loads keep the constant address space (scalar loads)
}

// A buffer kept as its base and extent, the descriptor rebuilt where it is used.  A kernel with
// many buffers live across its chunk loop holds four SGPRs per descriptor and spills them (every
// spilled SGPR costs a VALU lane write and read); the base takes two.  The empty asm makes the
// base opaque at each use, so the compiler cannot hoist the descriptor out of the loop.
struct RowRef {
  const char *base;
  int ext;
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc() const {
    const char *b = base;
    asm volatile("" : "+s"(b));
    return __builtin_amdgcn_make_buffer_rsrc((void *)b, (short)0, ext, kBufferFlags);
  }
};
// A row buffer read through windows that start a uniform byte offset into the row: a read at
// offset o of the window at `off` lands at row offset off + o and returns 0 past the row's extent,
// as through the whole row's buffer, while the chunk's offset costs a few scalar instructions
// (the window's base and extent) instead of a vector add per read.
struct RowWin {
  const char *base;
  int ext;
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t at(uint32_t off) const {
    const int rem = ext - (int)off;
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + off), (short)0, rem > 0 ? rem : 0, kBufferFlags);
  }
};
__device__ __forceinline__ RowWin row_win(const KView &V, int64_t b, int L, int C, int esize) {
  const int64_t ext = ((int64_t)(L - 1) * V.s1 + (int64_t)(C - 1) * V.s2 + 1) * esize;
  return RowWin{(const char *)V.p + b * V.s0 * esize, (int)ext};
}
__device__ __forceinline__ RowRef row_ref(const KView &V, int64_t b, int L, int C, int esize) {
  const int64_t ext = ((int64_t)(L - 1) * V.s1 + (int64_t)(C - 1) * V.s2 + 1) * esize;
  return RowRef{(const char *)V.p + b * V.s0 * esize, (int)ext};
}
__device__ __forceinline__ RowRef flat_ref(const void *base, int64_t bytes) {
  return RowRef{(const char *)base, (int)bytes};
}

// Byte offsets (at t0 = 0) of the tile elements a lane stages, for a view with element size `esize`.
template <int ROWS, int COLS, int E>
__device__ __forceinline__ void tile_offsets(uint32_t (&off)[E], const KView &V, int c0, bool tfast, int lane,
                                             int esize) {
#pragma unroll
  for (int i = 0; i < E; ++i) {
    int t, c;
    tc_of<ROWS, COLS>(lane + i * kWave, tfast, t, c);
    off[i] = (uint32_t)((t * (int)V.s1 + (c0 + c) * (int)V.s2) * esize);
  }
}

// Register staging of a CK x COLS tile of a (B, L, C) view for one wavefront.
// The loads are issued unconditionally from clamped (always valid) addresses and the
// out-of-range elements are zeroed only when the tile is stored to LDS: no branch surrounds a
// load, so the compiler can wait for one tile's loads (vmcnt(n)) while later prefetches and
// stores stay in flight, instead of draining the whole memory queue (vmcnt(0)).
template <typename IT, typename CT, int ROWS, int COLS, bool UL = false>
struct WaveTile {
  static constexpr int E = (ROWS * COLS + kWave - 1) / kWave;
  CT v[E];

  __device__ __forceinline__ void load(const KView &V, int64_t b, int t0, int L, int c0, int C, bool tfast,
                                       int lane) {
    const IT *base = (const IT *)V.p + b * V.s0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int e = lane + i * kWave;
      int t, c;
      tc_of<ROWS, COLS>(e, tfast, t, c);
      const int tc = min(t0 + t, L - 1), cc = min(c0 + c, C - 1);
      v[i] = Conv<IT>::load(base + row_off<UL>(tc, cc, V.s1, V.s2));
    }
  }

  // Buffer form of load(): `off` holds this lane's byte offsets at t0 = 0 (tile_offsets) and
  // `toff` the chunk's byte offset; reads past the row's extent return 0 and never fault.
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, const uint32_t (&off)[E], uint32_t toff) {
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = buf_load<IT>(r, off[i] + toff);
  }

  // Elements past the row's extent (t0 + t >= L or c0 + c >= C) are stored as 0; with RANGE
  // false the caller guarantees the whole tile lies inside (no range selects).
  template <bool RANGE = true, int RP>
  __device__ __forceinline__ void store(CT (*S)[RP], bool tfast, int lane, int t0, int L, int c0, int C) const {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int e = lane + i * kWave;
      if (e >= ROWS * COLS) break;
      int t, c;
      tc_of<ROWS, COLS>(e, tfast, t, c);
      S[c][t] = (!RANGE || (t0 + t < L && c0 + c < C)) ? v[i] : (CT)0;
    }
  }
  // The same elements stored step-major ([t][c]): a lane reads one step's values of every
  // column with 16-byte loads.
  template <bool RANGE = true, int RP>
  __device__ __forceinline__ void store_t(CT (*S)[RP], bool tfast, int lane, int t0, int L, int c0, int C) const {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int e = lane + i * kWave;
      if (e >= ROWS * COLS) break;
      int t, c;
      tc_of<ROWS, COLS>(e, tfast, t, c);
      S[t][c] = (!RANGE || (t0 + t < L && c0 + c < C)) ? v[i] : (CT)0;
    }
  }
};

// Per-lane delta bias of the tile elements a lane stages (the channel of element i of a lane is
// the same in every chunk), read once per kernel.
template <typename CT, int ROWS, int COLS, int E>
__device__ __forceinline__ void tile_bias(CT (&bv)[E], int has_bias, const KView &bias, int c0, int C, bool tfast,
                                          int lane) {
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int e = lane + i * kWave;
    int t, c;
    tc_of<ROWS, COLS>(e, tfast, t, c);
    bv[i] = (has_bias && e < ROWS * COLS && c0 + c < C) ? vload<CT>(bias, (int64_t)(c0 + c) * bias.s0) : (CT)0;
  }
}

// delta' = softplus(delta + bias) (optional parts) for in-range elements, padding stays 0;
// `sg` (optional) receives the softplus derivative sigmoid(delta + bias) (1 without softplus).
template <typename IT, typename CT, int ROWS, int COLS, int RP, bool UL>
__device__ __forceinline__ void store_delta_w(const WaveTile<IT, CT, ROWS, COLS, UL> &tl, CT (*S)[RP], CT (*sg)[RP],
                                              bool tfast, int lane, int softplus,
                                              const CT (&bv)[WaveTile<IT, CT, ROWS, COLS, UL>::E], int c0, int C,
                                              int t0, int L) {
#pragma unroll
  for (int i = 0; i < WaveTile<IT, CT, ROWS, COLS, UL>::E; ++i) {
    const int e = lane + i * kWave;
    if (e >= ROWS * COLS) break;
    int t, c;
    tc_of<ROWS, COLS>(e, tfast, t, c);
    CT v = 0, g = 1;
    if (t0 + t < L && c0 + c < C) {
      v = tl.v[i] + bv[i];
      if (softplus) {
        g = sigmoid_ct<CT>(v);
        v = softplus_ct<CT>(v);
      }
    }
    S[c][t] = v;
    if (sg) sg[c][t] = g;
  }
}

// Low-rank delta (the dt_proj GEMM of models/mamba.py:76 done in the staging).  A chunk's
// (CK, kLR) block of the (B, L, R) input, zero past R, is read E values per lane through a raw
// buffer over the batch row (reads past the row return 0; with lowrank off the buffer is empty
// and nothing is read), staged in LDS, and every staged (t, c) element of the delta tile is the
// dot product of input row t with channel c's weight row (in LDS for the whole kernel).
template <typename IT, typename CT, int CK>
struct LowRankTile {
  static constexpr int E = CK * kLR / kWave;
  static_assert(kWave % kLR == 0 && (CK * kLR) % kWave == 0, "low-rank tile shape");
  CT v[E];

  // lane element i is (t, r) = (lane / kLR + i * kWave / kLR, lane % kLR)
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rb, uint32_t off0, uint32_t tstep, bool rvalid) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const CT x = buf_load<IT>(rb, off0 + (uint32_t)i * tstep);
      v[i] = rvalid ? x : (CT)0;
    }
  }
  template <int RP>
  __device__ __forceinline__ void store(CT (*S)[RP], int lane) const {
#pragma unroll
    for (int i = 0; i < E; ++i) S[lane / kLR + i * (kWave / kLR)][lane % kLR] = v[i];
  }
};

// The lane's byte offset of element 0 of its low-rank block at t0 = 0, the step between its
// elements, and whether its rank index is below R.
__device__ __forceinline__ void lowrank_offsets(const KView &V, int R, int lane, int esize, uint32_t &off0,
                                                uint32_t &tstep, bool &rvalid) {
  const int r = lane % kLR, t = lane / kLR;
  rvalid = r < R;
  off0 = (uint32_t)((t * V.s1 + (r < R ? r : 0) * V.s2) * esize);
  tstep = (uint32_t)((kWave / kLR) * V.s1 * esize);
}

// The wavefront's channels' weight rows (D, R) into LDS, zero past R and past D.
template <typename CT, int COLS, int RP>
__device__ __forceinline__ void lowrank_weights(CT (*W)[RP], const KView &V, int R, int c0, int C, int lane) {
#pragma unroll
  for (int e = lane; e < COLS * kLR; e += kWave) {
    const int c = e / kLR, r = e % kLR;
    CT w = 0;
    if (r < R && c0 + c < C) w = vload<CT>(V, (int64_t)(c0 + c) * V.s0 + (int64_t)r * V.s1);
    W[c][r] = w;
  }
}

// Replaces the staged delta tile values by the projections: element (t, c) = sum_r in[t][r] W[c][r].
template <typename IT, typename CT, int ROWS, int COLS, bool UL, int RP>
__device__ __forceinline__ void lowrank_delta(WaveTile<IT, CT, ROWS, COLS, UL> &tl, const CT (*in)[RP],
                                              const CT (*W)[RP], bool tfast, int lane) {
#pragma unroll
  for (int i = 0; i < WaveTile<IT, CT, ROWS, COLS, UL>::E; ++i) {
    const int e = lane + i * kWave;
    if (e >= ROWS * COLS) break;
    int t, c;
    tc_of<ROWS, COLS>(e, tfast, t, c);
    CT a[kLR], w[kLR];
#pragma unroll
    for (int r = 0; r < kLR; ++r) {
      a[r] = in[t][r];
      w[r] = W[c][r];
    }
    CT acc = 0;
#pragma unroll
    for (int r = 0; r < kLR; ++r) acc = fma(a[r], w[r], acc);
    tl.v[i] = acc;
  }
}

// Waves per workgroup so that WPB copies of a per-wave LDS struct fit in 64 KiB.
template <int BYTES_PER_WAVE, int EXTRA = 0>
struct WavesPerBlock {
  static constexpr int fit = (64 * 1024 - EXTRA) / BYTES_PER_WAVE;
  static constexpr int value = fit >= 4 ? 4 : fit >= 2 ? 2 : 1;
};

}  // namespace ssm
