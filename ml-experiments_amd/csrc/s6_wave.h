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

__device__ inline float dpp_row_ror8(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x128, 0xf, 0xf, false));
}
__device__ inline float dpp_row_half_mirror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x141, 0xf, 0xf, false));
}
__device__ inline float dpp_quad_xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0xB1, 0xf, 0xf, false));
}
__device__ inline float dpp_quad_xor2(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x4E, 0xf, 0xf, false));
}

// Sum v[n] over the 64 lanes of the wave for n = 0..15.  On return every lane l holds in
// v[0] the sum for n = l / 4 (each group of 4 lanes holds the same value).
__device__ inline void wave_transpose_reduce16(float (&v)[16], int lane) {
  // lanes l and l^32: swap halves of (v[i], v[i+8]) -> low half keeps n=i, high n=i+8
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    permlane32_swap(v[i], v[i + 8]);
    v[i] = v[i] + v[i + 8];
  }
  // lanes l and l^16: row r keeps n = 4r + i for i < 4
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    permlane16_swap(v[i], v[i + 4]);
    v[i] = v[i] + v[i + 4];
  }
  // lanes l and l^8 inside a row: the low 8 lanes keep i, the high 8 keep i + 2
  const bool hi8 = (lane & 8) != 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float send = hi8 ? v[i] : v[i + 2];
    float keep = hi8 ? v[i + 2] : v[i];
    v[i] = keep + dpp_row_ror8(send);
  }
  // lanes l and 7-l inside each 8-lane half: the low 4 keep v[0], the high 4 keep v[1]
  {
    const bool hi4 = (lane & 4) != 0;
    float send = hi4 ? v[0] : v[1];
    float keep = hi4 ? v[1] : v[0];
    v[0] = keep + dpp_row_half_mirror(send);
  }
  v[0] += dpp_quad_xor1(v[0]);
  v[0] += dpp_quad_xor2(v[0]);
}


}  // namespace s6
