// Cross-lane helpers for 64-lane wavefronts on gfx950 (permlane swaps and DPP).
#pragma once
#include <hip/hip_runtime.h>

namespace s6 {

// v_permlane32_swap_b32 a, b: afterwards a = [a.lo32, b.lo32] and b = [a.hi32, b.hi32]
// (lanes 0-31 | 32-63).  v_permlane16_swap_b32 a, b exchanges the odd 16-lane rows of a
// with the even rows of b: a = [a.r0, b.r0, a.r2, b.r2], b = [a.r1, b.r1, a.r3, b.r3].
// Issued through inline asm because the clang builtins of this toolchain return the first
// register for both results.  The s_nop pads cover VALU-write -> permlane-read and
// permlane-write -> VALU-read forwarding on gfx950.
__device__ inline void permlane32_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ inline void permlane16_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// DPP lane permutations within 16-lane rows.  Each one is a full permutation (every lane
// reads a valid source), so bound_ctrl is set and the move can fold into the consuming add.
__device__ inline float dpp_row_ror8(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x128, 0xf, 0xf, true));
}
__device__ inline float dpp_row_half_mirror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x141, 0xf, 0xf, true));
}
__device__ inline float dpp_quad_xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0xB1, 0xf, 0xf, true));
}
__device__ inline float dpp_quad_xor2(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x4E, 0xf, 0xf, true));
}

// Sum v[n] over the 64 lanes of the wave for n = 0..7.  On return v[0] on lane l holds the
// sum for n = (l >> 3) & 7 (each group of 8 consecutive lanes holds the same value).
// 4 + 2 permlane swaps, 2 selects and 7 adds for 8 sums.
__device__ inline void wave_transpose_reduce8(float (&v)[8], int lane) {
  // lanes l and l^32: the low half keeps n = i, the high half n = i + 4
  asm volatile(
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %4\n\t"
      "v_permlane32_swap_b32 %1, %5\n\t"
      "v_permlane32_swap_b32 %2, %6\n\t"
      "v_permlane32_swap_b32 %3, %7\n\t"
      "s_nop 1"
      : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),
        "+v"(v[7]));
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] += v[i + 4];
  // lanes l and l^16: row r keeps n = i + 2 (r & 1) + 4 (r >> 1) for i < 2
  asm volatile(
      "s_nop 1\n\t"
      "v_permlane16_swap_b32 %0, %2\n\t"
      "v_permlane16_swap_b32 %1, %3\n\t"
      "s_nop 1"
      : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
  v[0] += v[2];
  v[1] += v[3];
  // lanes l and l^8 inside a row: the low 8 lanes keep i = 0, the high 8 keep i = 1
  const bool hi8 = (lane & 8) != 0;
  const float send = hi8 ? v[0] : v[1];
  const float keep = hi8 ? v[1] : v[0];
  v[0] = keep + dpp_row_ror8(send);
  // sum over the 8 lanes of each half-row (bits 0-2 of the lane)
  v[0] += dpp_quad_xor1(v[0]);
  v[0] += dpp_quad_xor2(v[0]);
  v[0] += dpp_row_half_mirror(v[0]);
}

}  // namespace s6
