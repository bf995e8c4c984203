// Cross-lane sums and moves on the VALU (DPP and v_permlane*_swap) for the
// element-wise kernels, in place of LDS-routed shuffles. Every helper reads
// other lanes, so it must run with every lane of the wave active.
#pragma once

#include "inl_common.hpp"

namespace inl {

// dpp<CTRL>(x): lane i reads the lane that CTRL names within its row of 16
// (quad_perm 0x00-0xFF, row_shl 0x101-0x10F, row_shr 0x111-0x11F, row_ror
// 0x121-0x12F, row_mirror 0x140, row_half_mirror 0x141); a lane outside the
// row reads 0.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum of x over each aligned group of G lanes (G a power of two <= 64), in
// every lane of the group: pairs, quads, mirrored halves and mirrored rows by
// DPP, then v_permlane16_swap and v_permlane32_swap across rows.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (G >= 2) x += dpp<0xB1>(x);     // quad_perm [1, 0, 3, 2]
  if constexpr (G >= 4) x += dpp<0x4E>(x);     // quad_perm [2, 3, 0, 1]
  if constexpr (G >= 8) x += dpp<0x141>(x);    // row_half_mirror: quad q <-> quad 1 - q of each 8
  if constexpr (G >= 16) x += dpp<0x140>(x);   // row_mirror: 8-lane halves of each row
  if constexpr (G >= 32) {
    float a = x, b = x;   // a: rows (0, 0, 2, 2), b: rows (1, 1, 3, 3)
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    x = a + b;
  }
  if constexpr (G >= 64) {
    float a = x, b = x;   // a: halves (0, 0), b: halves (1, 1)
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    x = a + b;
  }
  return x;
}

__device__ __forceinline__ float wave_sum(float x) { return group_sum<64>(x); }

}  // namespace inl
