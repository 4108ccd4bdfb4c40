// Register tiles of per-(step, channel) values delivered to the lanes by DPP row broadcasts.
//
// The fused float kernels give each 64-lane wavefront CW = 64 / NP channels of one batch row,
// one lane per (channel, state): channel c owns the RPC = NP / 16 consecutive 16-lane rows
// starting at row c * RPC.  A chunk's per-(step, channel) inputs (x, delta, the gate, dy) are
// held one value per lane in a "row tile": lane (row r, position j) holds the value of step j
// for the channel that owns row r.  Step t of the chunk then reaches every lane of the channel
// as the DPP source modifier row_newbcast:t on the instruction that consumes it (gfx90a and
// later), so these inputs never pass through LDS.  Outputs per (step, channel) (dx, ddelta,
// the scan output) come back in the same layout: lane (r, j) owns step j of its channel, and
// the first row of each channel stores it.
#pragma once

#include <type_traits>

#include "ssm_device.hpp"
#include "ssm_internal.hpp"
#include "ssm_tiles.hpp"
#include "ssm_wave.hpp"

namespace ssm {

constexpr int kRow = 16;  // lanes per DPP row

// Value of lane `T` of this lane's 16-lane row.
template <int T>
__device__ __forceinline__ float row_bcast(float v) {
  static_assert(T >= 0 && T < kRow, "row lane");
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + T, 0xF, 0xF, true));
}

// Row shifts by 8 lanes (lanes shifted in from outside the row read 0).
__device__ __forceinline__ float row_shr8(float v) {  // lane i gets lane i - 8
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x118, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_shl8(float v) {  // lane i gets lane i + 8
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x108, 0xF, 0xF, true));
}
// Sum over the 16 lanes of a row, every lane receiving the same bits (fixed order).
__device__ __forceinline__ float row_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

// The same row sum in float64 (the two halves of each value move by the same DPP pattern).
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xF, 0xF, false);
  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double row_sum_f64(double v) {
  v += dpp_d<0xB1>(v);
  v += dpp_d<0x4E>(v);
  v += dpp_d<0x141>(v);
  v += dpp_d<0x140>(v);
  return v;
}

// Scheduling ties (no instructions): `order_after(a, b)` makes the compiler treat `a` as
// rewritten from `b`, so every later use of `a` is scheduled after `b` is computed.  The
// software-pipelined kernels use them to keep a serial recurrence interleaved step by step
// with independent work, which the scheduler would otherwise cluster.
__device__ __forceinline__ void order_after(float &a, float b) { asm volatile("" : "+v"(a) : "v"(b)); }
__device__ __forceinline__ void order_after(float &a, float b, float c) { asm volatile("" : "+v"(a) : "v"(b), "v"(c)); }

// Calls f(std::integral_constant<int, I>) for I = B .. E-1 in order (every I a compile-time
// constant, as the DPP controls require).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}
template <int B, int E, typename F>
__device__ __forceinline__ void static_for_down(F &&f) {  // I = E-1 .. B
  if constexpr (B < E) {
    f(std::integral_constant<int, E - 1>{});
    static_for_down<B, E - 1>(f);
  }
}

// Geometry of a row tile for NP states per channel.
template <int NP>
struct RowGeo {
  static_assert(NP >= kRow && NP <= kWave, "row tiles need 16..64 states per channel");
  static constexpr int CW = kWave / NP;    // channels per wavefront
  static constexpr int RPC = NP / kRow;    // rows per channel
  __device__ __forceinline__ static int step(int lane) { return lane % kRow; }
  __device__ __forceinline__ static int chan(int lane) { return lane / kRow / RPC; }
  // true on the lanes that store a channel's per-step outputs (its first row)
  __device__ __forceinline__ static bool lead(int lane) { return (lane / kRow) % RPC == 0; }
};

// One row tile of a (B, L, C) view: lane -> (step j, channel c) = (lane % 16, chan(lane)).
template <typename IT, int NP, bool UL>
struct RowTile {
  typedef RowGeo<NP> G;
  float v;

  // Byte offset (step 0 of the chunk) of this lane's element, for the raw-buffer reads.
  __device__ __forceinline__ static uint32_t offset(const KView &V, int c0, int lane) {
    return (uint32_t)((G::step(lane) * (int)V.s1 + (c0 + G::chan(lane)) * (int)V.s2) * (int)sizeof(IT));
  }
  // Raw-buffer read: reads past the row's extent return 0 and never fault.
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t toff) {
    v = buf_load<IT>(r, off + toff);
  }
  // Strided read from a clamped (always valid) address.
  __device__ __forceinline__ void load(const KView &V, int64_t b, int t0, int L, int c0, int C, int lane) {
    const int t = min(t0 + G::step(lane), L - 1), c = min(c0 + G::chan(lane), C - 1);
    v = Conv<IT>::load((const IT *)V.p + b * V.s0 + (int64_t)t * V.s1 + (int64_t)c * V.s2);
  }
};

}  // namespace ssm
