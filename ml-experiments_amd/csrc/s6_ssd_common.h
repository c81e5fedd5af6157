// Shared device code of the Mamba-2 SSD kernels (s6_ssd.hip forward, s6_ssd_bwd.hip
// backward): the MFMA operand abstraction and small helpers.
//
// MFMA use.  Every contraction runs on 16x16 output tiles with K = 32 per step: one
// v_mfma_f32_16x16x32_bf16 / _f16 for bf16 / fp16 operands, eight v_mfma_f32_16x16x4_f32
// for fp32.
// Lane i of a wave holds A[i % 16][k(i, j)] and B[k(i, j)][i % 16] for items j < 8, with
// k(i, j) = 8 (i / 16) + j (bf16, fp16) or i / 16 + 4 j (fp32), and D[4 (i / 16) + j][i % 16]
// for j < 4.
#pragma once
#include "s6_internal.h"
#include "ssd.h"

namespace s6 {
namespace ssd {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));  // 16 raw bytes (kept in registers)
constexpr int kKs = 32;            // sequence steps per MFMA K step (and per LDS slice)
constexpr int kLp = kKs + 8;       // LDS row pitch in elements: 16-byte aligned rows
constexpr int kThreads = 256;

template <typename T> struct Mma;
// 16-bit operand types (bf16, fp16): 8 elements of one row per lane, one 16-byte load.
template <typename E>
struct Mma16 {
  typedef E Frag __attribute__((ext_vector_type(8)));
  typedef uint16_t Raw;
  static constexpr int kVe = 8;  // elements per 16-byte load
  __device__ static inline int kidx(int lane, int j) { return 8 * (lane >> 4) + j; }
  __device__ static inline Frag load_row(const Raw* row_k0, int lane) {
    return *reinterpret_cast<const Frag*>(row_k0 + 8 * (lane >> 4));
  }
  // Operand fragment of the 16 columns starting at tile[0][0] over K = 32 rows of a
  // row-major LDS tile (K along rows, pitch in elements, rows 8-byte aligned), through
  // gfx950's transposing LDS read.  ds_read_b64_tr_b16 returns to lane i of each 16-lane
  // group element i % 4 of the 8-byte chunks addressed by lanes 4 j + i / 4 (j < 4), as
  // measured on the device; so lane 16 g + s addresses row 8 g + 4 h + s / 4, column
  // 4 (s % 4), and the reads h = 0, 1 return this lane's k = 8 g + 4 h .. + 3.
  __device__ static inline Frag load_tr(const Raw* tile, int pitch, int lane) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    const int g = lane >> 4, s = lane & 15;
    const Raw* p0 = tile + (8 * g + (s >> 2)) * pitch + 4 * (s & 3);
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4s*)(p0));
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4s*)(p0 + 4 * pitch));
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(Frag, both);
  }
  __device__ static inline Frag from_float(const float (&v)[8]) {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = static_cast<E>(v[j]);
    return f;
  }
  __device__ static inline Frag zero() {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = static_cast<E>(0.f);
    return f;
  }
  __device__ static inline Raw to_raw(float v) { return __builtin_bit_cast(uint16_t, static_cast<E>(v)); }
  __device__ static inline float from_raw(Raw r) { return static_cast<float>(__builtin_bit_cast(E, r)); }
};
template <> struct Mma<bf16> : Mma16<__bf16> {
  __device__ static inline void mma(f4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  __device__ static inline float from_raw(Raw r) { return __uint_as_float((uint32_t)r << 16); }
};
template <> struct Mma<f16> : Mma16<_Float16> {
  __device__ static inline void mma(f4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
  }
};
template <> struct Mma<float> {
  struct Frag { float v[8]; };
  typedef float Raw;
  static constexpr int kVe = 4;
  __device__ static inline int kidx(int lane, int j) { return (lane >> 4) + 4 * j; }
  __device__ static inline Frag load_row(const Raw* row_k0, int lane) {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = row_k0[(lane >> 4) + 4 * j];
    return f;
  }
  __device__ static inline Frag from_float(const float (&v)[8]) {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = v[j];
    return f;
  }
  __device__ static inline Frag zero() {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = 0.f;
    return f;
  }
  __device__ static inline void mma(f4& acc, const Frag& a, const Frag& b) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[j], b.v[j], acc, 0, 0, 0);
  }
  __device__ static inline Raw to_raw(float v) { return v; }
  __device__ static inline float from_raw(Raw r) { return r; }
};

// 16 bytes of a row, as kVe raw elements.
template <typename T>
__device__ inline void load16(const void* p, typename Mma<T>::Raw (&r)[Mma<T>::kVe]) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  *reinterpret_cast<uint4*>(r) = v;
}

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2.  This maps
// the linear workgroup id to a work id so that each XCD runs one contiguous range of work
// ids (a bijection for any grid size): blocks that share tiles -- the heads and row tiles
// of one (batch, chunk) -- then share one L2.
__device__ inline int64_t xcd_work_id() {
  const int64_t n = gridDim.x, id = blockIdx.x;
  const int64_t x = id & 7, loc = id >> 3, q = n >> 3, r = n & 7;
  return x * q + (x < r ? x : r) + loc;
}

__device__ inline int32_t seq_at(const SsdK& k, int64_t b, int64_t t) {
  return k.seq[b * k.sseq[0] + t * k.sseq[1]];
}

}  // namespace ssd
}  // namespace s6
