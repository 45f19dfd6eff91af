// Shared device/host helpers of libxenc_hip.so (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/xenc_hip.h"

namespace xenc {

constexpr int kWave = 64;

// Error state of the last failed launch on this host thread.
void set_hip_error(hipError_t e);

inline int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_hip_error(e);
    return XENC_EHIP;
  }
  return XENC_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The most LDS (static + dynamic) one workgroup may use on the current device, queried once per
// device (64 KiB if the query fails).
inline size_t device_lds_limit() {
  constexpr int kDevices = 64;
  static int cached[kDevices];  // 0 = not yet queried
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevices) return 64 * 1024;
  int v = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
      v = 64 * 1024;
    __atomic_store_n(&cached[dev], v, __ATOMIC_RELAXED);
  }
  return (size_t)v;
}

// ---------------------------------------------------------------- wave-level primitives
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ __forceinline__ int shfl_xor(int v, int mask) { return __shfl_xor(v, mask, kWave); }

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// DPP move of x with the given control (row_mask / bank_mask all, bound_ctrl on): a VALU
// operand, no LDS-pipe permute.
//
// Precondition of every reduction built on it (dpp_f, swap_partner, group_sum, wave_sum,
// wave_max, wave_reduce_scatter): ALL 64 lanes of the wave are active.  With bound_ctrl on, an
// inactive source lane reads as 0, and the permlane swaps move whatever the inactive lanes hold,
// so a partial wave would add zeros to a sum or raise a max of negative values to 0.  Callers
// reach these helpers only with wave-uniform control flow (whole waves exit early or not at
// all).  Debug builds (XENC_CHECK_FULL_WAVE) trap when the precondition is broken.
__device__ __forceinline__ void assert_full_wave() {
#ifdef XENC_CHECK_FULL_WAVE
  if (__builtin_amdgcn_read_exec() != ~0ull) __builtin_trap();
#endif
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  assert_full_wave();
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// The value of lane ^ MASK (MASK 32 or 16) by the gfx950 permlane swaps.  hi = (lane & MASK) != 0.
// permlane32_swap exchanges lanes 32-63 of its first operand with lanes 0-31 of its second
// (permlane16_swap: the odd 16-lane rows with the even rows), so with x in both the first result
// holds the partner's value in the upper lanes and the second in the lower lanes.
template <int MASK>
__device__ __forceinline__ float swap_partner(float x, bool hi) {
  static_assert(MASK == 32 || MASK == 16, "permlane swaps pair lanes at distance 32 or 16");
  assert_full_wave();
  const unsigned u = __float_as_uint(x);
  if constexpr (MASK == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(hi ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(hi ? r[0] : r[1]);
  }
}

// Sum over each aligned group of TPR lanes (a power of two <= 64), every lane of the group ending
// with the same bits.  Inside a 16-lane row the partner values come by DPP (quad xor 1, xor 2,
// half-row mirror, row mirror), across rows by the permlane swaps, so the VALU does the whole
// reduction.  Each step adds the two halves in the same order in both lanes of a pair.
template <int TPR>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (TPR >= 2) v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
  if constexpr (TPR >= 4) v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
  if constexpr (TPR >= 8) v += dpp_f<0x141>(v);   // row_half_mirror: the other quad of the 8
  if constexpr (TPR >= 16) v += dpp_f<0x140>(v);  // row_mirror: the other 8 of the row
  if constexpr (TPR >= 32) {                    // rows 2i, 2i+1: (even row) + (odd row) in both
    const unsigned u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (TPR >= 64) {                    // lanes 0-31 + lanes 32-63 in both halves
    const unsigned u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return v;
}

// Sum and max over the wave, every lane ending with the result: inside each 16-lane row by DPP,
// across rows by the permlane swaps, so the reduction stays on the VALU (no LDS-pipe permutes).
// A fixed order: deterministic.
__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));    // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f<0x141>(v));   // row_half_mirror
  v = fmaxf(v, dpp_f<0x140>(v));   // row_mirror
  unsigned u = __float_as_uint(v);
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  u = __float_as_uint(v);
  r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Reduce SPT per-lane partial values over the 64 lanes.  On return v[0] holds, in every lane,
// the full sum for slot j = lane / (64 / SPT).  Step with lane bit MASK: lanes with the bit set
// keep the upper half of the remaining values, send the lower half to their partner and add
// what they receive.  The steps at lane distance 32 and 16 go through the permlane swaps; once
// one value is left at distance 8, the 16-lane row is summed by DPP.  Written as compile-time
// recursion so every array index is a constant.
template <int SPT, int CNT = SPT, int MASK = 32>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[SPT], int lane) {
  static_assert(SPT >= 1 && SPT <= 64 && (SPT & (SPT - 1)) == 0, "SPT must be a power of 2");
  if constexpr (CNT > 1) {
    constexpr int H = CNT / 2;
    const bool hi = (lane & MASK) != 0;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float send = hi ? v[i] : v[i + H];
      const float keep = hi ? v[i + H] : v[i];
      if constexpr (MASK >= 16) {
        v[i] = keep + swap_partner<MASK>(send, hi);
      } else {
        v[i] = keep + shfl_xor(send, MASK);
      }
    }
    wave_reduce_scatter<SPT, H, MASK / 2>(v, lane);
  } else if constexpr (MASK >= 16) {
    v[0] += swap_partner<MASK>(v[0], (lane & MASK) != 0);
    wave_reduce_scatter<SPT, 1, MASK / 2>(v, lane);
  } else if constexpr (MASK == 8) {
    v[0] = group_sum<16>(v[0]);
  } else if constexpr (MASK >= 1) {
    v[0] += shfl_xor(v[0], MASK);
    wave_reduce_scatter<SPT, 1, MASK / 2>(v, lane);
  }
}

// (value, index) order used by every top-k here: larger value first, then lower index.
__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// Order key of a logit: unsigned integers compare as the floats do, -0 is folded onto +0 (the
// reference's == ties them) and every NaN onto one key above +inf (topk ranks NaN first).
__device__ __forceinline__ unsigned order_key(float x) {
  if (x == 0.f) x = 0.f;
  if (x != x) x = __uint_as_float(0x7fc00000u);
  const unsigned b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).  Tile b is
// remapped so that XCD x runs a contiguous range of logical tiles; the logical order then puts
// tiles that share operands next to each other, so the workgroups resident on one XCD at a time
// hit in that XCD's L2 instead of re-reading HBM.  A bijection on [0, n).
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_remap(int b, int n) {
  const int x = b % kXcds, j = b / kXcds;
  const int per = (n + kXcds - 1) / kXcds, rem = n % kXcds;
  const int start = rem == 0 ? x * per : x * per - max(0, x - rem);
  return start + j;
}

}  // namespace xenc
