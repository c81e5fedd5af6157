// Shared definitions for the gfx950 S6 selective-scan kernels (device side and host side).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "s6scan.h"

namespace s6 {

constexpr int kWave = 64;            // CDNA wavefront width
constexpr int kCk = S6_CKPT_INTERVAL;
constexpr float kLog2e = 1.4426950408889634f;

// Element storage types (tags; raw bits for the 16-bit formats).
struct bf16 { uint16_t bits; };
struct f16 { uint16_t bits; };

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kSize = 4;
  __device__ static inline float load(const void* p, int64_t i) {
    return reinterpret_cast<const float*>(p)[i];
  }
  __device__ static inline void store(void* p, int64_t i, float v) {
    reinterpret_cast<float*>(p)[i] = v;
  }
};
template <> struct Elem<bf16> {
  static constexpr int kSize = 2;
  __device__ static inline float load(const void* p, int64_t i) {
    uint32_t b = reinterpret_cast<const uint16_t*>(p)[i];
    return __uint_as_float(b << 16);
  }
  __device__ static inline void store(void* p, int64_t i, float v) {
    // gfx950 converts f32 -> bf16 with round-to-nearest-even in hardware.
    __bf16 h = static_cast<__bf16>(v);
    reinterpret_cast<__bf16*>(p)[i] = h;
  }
};
template <> struct Elem<f16> {
  static constexpr int kSize = 2;
  __device__ static inline float load(const void* p, int64_t i) {
    return static_cast<float>(reinterpret_cast<const _Float16*>(p)[i]);
  }
  __device__ static inline void store(void* p, int64_t i, float v) {
    asm("" : "+v"(v));  // rounded to fp32 first (see Buf<f16>::store)
    reinterpret_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  }
};

// Raw buffer access.  Each wave addresses its tensors through a buffer resource whose base
// is the wave's first element; a lane's channel offset goes in the VGPR offset and the time
// offset, identical for all lanes, in the SGPR offset, so stepping in time costs no VALU
// address arithmetic.  Lanes past the last channel get kOffDrop: their loads return 0 and
// their stores are dropped by the buffer range check (num_records = kBufRecords).
constexpr uint32_t kBufRecords = 0x7fffffffu;
constexpr uint32_t kOffDrop = 0x80000000u;
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)kBufRecords,
                                           0x00020000);
}

// load_raw / from_raw: a prefetched value carried into a later loop iteration stays as its
// raw bits until used.  Converted right after its load (as load() does), it would make the
// prefetch wait for the load in the iteration that issues it.
template <typename T> struct Buf;
template <> struct Buf<float> {
  __device__ static inline float load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0));
  }
  __device__ static inline uint32_t load_raw(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0);
  }
  __device__ static inline float from_raw(uint32_t x) { return __uint_as_float(x); }
  __device__ static inline void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)vo, (int)so, 0);
  }
};
template <> struct Buf<bf16> {
  __device__ static inline float load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    const uint32_t b = __builtin_amdgcn_raw_buffer_load_b16(r, (int)vo, (int)so, 0);
    return __uint_as_float(b << 16);
  }
  __device__ static inline uint32_t load_raw(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)vo, (int)so, 0);
  }
  __device__ static inline float from_raw(uint32_t x) { return __uint_as_float(x << 16); }
  __device__ static inline void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float v) {
    const uint16_t b = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    __builtin_amdgcn_raw_buffer_store_b16(b, r, (int)vo, (int)so, 0);
  }
};
template <> struct Buf<f16> {
  __device__ static inline float load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    const uint16_t b = __builtin_amdgcn_raw_buffer_load_b16(r, (int)vo, (int)so, 0);
    return (float)__builtin_bit_cast(_Float16, b);
  }
  __device__ static inline uint32_t load_raw(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)vo, (int)so, 0);
  }
  __device__ static inline float from_raw(uint32_t x) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)x);
  }
  // The value is rounded to fp32 first, as the reference converts its fp32 results: the
  // empty asm stops the compiler from fusing a producing fma into v_fma_mixlo_f16, which
  // rounds once, straight to fp16 (one ulp apart now and then).
  __device__ static inline void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float v) {
    asm("" : "+v"(v));
    const uint16_t b = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    __builtin_amdgcn_raw_buffer_store_b16(b, r, (int)vo, (int)so, 0);
  }
};

// Row8<T>: eight consecutive time steps of one lane's row, packed in the storage format (two
// 16-bit values per word).  load() / store() move a whole block with 16-byte buffer accesses
// (one for the 16-bit formats, two for fp32): for a tensor whose time axis is contiguous and
// 16-byte aligned at every block of 8 steps, this replaces eight per-step accesses, each of
// which touches one cache line per lane.  pack() rounds to the storage format as the
// per-step store() does (round to nearest even), set2(k, ., .) steps 2k and 2k + 1;
// settle() is an empty asm that reads the words, so that their load completes there.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <typename T> struct Row8;
template <> struct Row8<float> {
  u32x4 w[2];
  __device__ inline void load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)so, 0);
    w[1] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)(so + 16), 0);
  }
  __device__ inline void settle() const { asm volatile("" ::"v"(w[0]), "v"(w[1])); }
  __device__ inline float get(int i) const { return __uint_as_float(w[i >> 2][i & 3]); }
  __device__ inline void set2(int k, float y0, float y1) {
    w[k >> 1][(k & 1) * 2] = __float_as_uint(y0);
    w[k >> 1][(k & 1) * 2 + 1] = __float_as_uint(y1);
  }
  __device__ inline void pack(const float (&y)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) set2(k, y[2 * k], y[2 * k + 1]);
  }
  __device__ inline void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) const {
    __builtin_amdgcn_raw_buffer_store_b128(w[0], r, (int)vo, (int)so, 0);
    __builtin_amdgcn_raw_buffer_store_b128(w[1], r, (int)vo, (int)(so + 16), 0);
  }
};
template <> struct Row8<bf16> {
  u32x4 w;
  __device__ inline void load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    w = __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)so, 0);
  }
  __device__ inline void settle() const { asm volatile("" ::"v"(w)); }
  __device__ inline float get(int i) const {
    const uint32_t x = w[i >> 1];
    return __uint_as_float((i & 1) ? (x & 0xffff0000u) : (x << 16));
  }
  __device__ inline void set2(int k, float y0, float y1) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){y0, y1}, bf16x2));
  }
  __device__ inline void pack(const float (&y)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) set2(k, y[2 * k], y[2 * k + 1]);
  }
  __device__ inline void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) const {
    __builtin_amdgcn_raw_buffer_store_b128(w, r, (int)vo, (int)so, 0);
  }
};
template <> struct Row8<f16> {
  u32x4 w;
  __device__ inline void load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    w = __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)so, 0);
  }
  __device__ inline void settle() const { asm volatile("" ::"v"(w)); }
  __device__ inline float get(int i) const {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i >> 1] >> ((i & 1) * 16)));
  }
  __device__ inline void set2(int k, float y0, float y1) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){y0, y1}, f16x2));
  }
  __device__ inline void pack(const float (&y)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) set2(k, y[2 * k], y[2 * k + 1]);
  }
  __device__ inline void store(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) const {
    __builtin_amdgcn_raw_buffer_store_b128(w, r, (int)vo, (int)so, 0);
  }
};

// Uniform (wave-invariant) loads of B_t / C_t through the scalar cache.  The pointer is
// cast to the constant address space so a uniform address is selected as s_load; the
// 16-bit formats are loaded as packed 32-bit pairs and unpacked on the scalar unit.
typedef const __attribute__((address_space(4))) uint32_t* cu32p;

// An empty asm that reads 8 SGPR words: the compiler must complete their loads before it.
__device__ inline void touch_words(const uint32_t (&w)[8]) {
  asm volatile("" ::"s"(w[0]), "s"(w[1]), "s"(w[2]), "s"(w[3]), "s"(w[4]), "s"(w[5]), "s"(w[6]),
               "s"(w[7]));
}

// A group of up to 16 consecutive states of one B or C row, as raw 32-bit words in SGPRs.
// The 16-bit formats stay packed two per word until the value is used.
template <typename T> struct BCGroup;
template <> struct BCGroup<float> {
  static constexpr int kWords = 8;
  uint32_t w[8];
  template <int G>
  __device__ inline void load(const char* row) {
    cu32p r = (cu32p)row;
#pragma unroll
    for (int i = 0; i < G; ++i) w[i] = r[i];
  }
  __device__ inline float get(int n) const { return __uint_as_float(w[n]); }
  __device__ inline void touch() const { touch_words(w); }
};
template <> struct BCGroup<bf16> {
  static constexpr int kWords = 8;
  uint32_t w[8];
  template <int G>
  __device__ inline void load(const char* row) {
    cu32p r = (cu32p)row;
#pragma unroll
    for (int i = 0; i < G / 2; ++i) w[i] = r[i];
  }
  __device__ inline float get(int n) const {
    const uint32_t x = w[n >> 1];
    return (n & 1) ? __uint_as_float(x & 0xffff0000u) : __uint_as_float(x << 16);
  }
  __device__ inline void touch() const { touch_words(w); }
};
template <> struct BCGroup<f16> {
  static constexpr int kWords = 8;
  uint32_t w[8];
  template <int G>
  __device__ inline void load(const char* row) {
    cu32p r = (cu32p)row;
#pragma unroll
    for (int i = 0; i < G / 2; ++i) w[i] = r[i];
  }
  __device__ inline float get(int n) const {
    const uint32_t x = w[n >> 1];
    return (float)__builtin_bit_cast(_Float16, (uint16_t)((n & 1) ? (x >> 16) : (x & 0xffffu)));
  }
  __device__ inline void touch() const { touch_words(w); }
};

// Whole-row loads (NS values) for the backward kernels.
template <typename T> struct BCLoad {
  template <int NS>
  __device__ static inline void row(const void* row, float (&v)[NS]) {
    static_assert(NS % 16 == 0 || NS < 16, "row width");
    constexpr int G = NS < 16 ? NS : 16;
#pragma unroll
    for (int g0 = 0; g0 < NS; g0 += G) {
      BCGroup<T> grp;
      grp.template load<G>((const char*)row + g0 * Elem<T>::kSize);
#pragma unroll
      for (int n = 0; n < G; ++n) v[g0 + n] = grp.get(n);
    }
  }
};

// States of one B/C row that one scalar group (8 words, s_load_dwordx8) holds.
template <typename T> constexpr int kGroupStates = 32 / Elem<T>::kSize;

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2eLo = 1.925963033500011e-08f;  // log2(e) - (float)log2(e)
constexpr float kLn2 = 0.69314718055994531f;

// e^x from the hardware exp2 with the exponent x log2(e) carried as hi + lo, so the
// rounding of the product does not reach the result (a few ulp for |x| < 88).
__device__ inline float exp_split(float x) {
  const float p = x * kLog2e;
  const float lo = fmaf(x, kLog2eLo, fmaf(x, kLog2e, -p));
  const float e = fast_exp2(p);
  return fmaf(e, lo * kLn2, e);
}

// F.softplus with beta=1, threshold=20 (selective_scan_interface.py:111-112): x above 20,
// else log(1 + e^x), evaluated as max(x, 0) + log1p(e^-|x|) with the hardware log2 and
// log1p(t) = ln(u) t / (u - 1), u = 1 + t, which cancels the rounding of 1 + t.  Within
// 4 ulp of torch's fp32 softplus (float32 emulation over 3e5 points in [-30, 25]).
__device__ inline float softplus20(float x) {
  const float t = exp_split(-fabsf(x));
  const float u = 1.f + t;
  const float um1 = u - 1.f;
  const float lp =
      um1 == 0.f ? t : (__builtin_amdgcn_logf(u) * kLn2) * (t * __builtin_amdgcn_rcpf(um1));
  const float sp = fmaxf(x, 0.f) + lp;
  return x > 20.f ? x : sp;
}
// d softplus / dx as torch's softplus_backward: e^x / (e^x + 1) below the threshold, else 1.
__device__ inline float softplus20_grad(float x) {
  const float e = exp_split(fminf(x, 20.f));
  const float g = e * __builtin_amdgcn_rcpf(e + 1.f);
  return x > 20.f ? 1.f : g;
}
// 1 / (1 + e^-x)  (silu(z) = z sigmoid(z), SSI:154-155)
__device__ inline float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.f + exp_split(-x));
}

// How Delta is formed from the delta input (selective_scan_interface.py:107-112): as is,
// plus delta_bias, or softplus(delta + delta_bias) (bias 0 when absent).
enum DtMode { kDtRaw = 0, kDtBias = 1, kDtSoftplus = 2 };
inline int dt_mode(int has_bias, int softplus) {
  return softplus ? kDtSoftplus : (has_bias ? kDtBias : kDtRaw);
}
template <int DTM>
__device__ inline float prep_dt(float raw, float bias) {
  if constexpr (DTM == kDtRaw) return raw;
  else if constexpr (DTM == kDtBias) return raw + bias;
  else return softplus20(raw + bias);
}

// Scalar-load pipelining.  Scalar loads complete out of order, so the compiler can only
// wait for all of them (lgkmcnt(0)); and loads from the constant address space are
// invariant, so LLVM may hoist the next row's load above the point where the current row
// is first consumed -- which makes every wait cover a load that was just issued.  The
// pattern used by the scans is therefore
//     cur.touch();                 // consume the group in flight: the compiler waits here
//     off = opaque(off);           // the next address is only known after that point
//     nxt.load(base + off);        // ... so the next load is issued after the wait
// which leaves one group of compute between a load and its wait.
__device__ inline uint32_t opaque(uint32_t x) {
  asm volatile("" : "+s"(x));
  return x;
}

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X, each with its own
// L2.  The kernels take a 1-D grid and remap the linear id so that consecutive logical
// blocks -- the channel blocks of one (batch, chunk), which read the same B/C rows --
// run on the same XCD.  Logical block = (x, y) with x fastest, x < nx.
struct BlockPos {
  int64_t x, y;
};
__device__ inline BlockPos block_pos(int64_t nx) {
  const int64_t total = gridDim.x;
  int64_t id = blockIdx.x;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  return {id % nx, id / nx};
}
inline dim3 xcd_grid(int64_t nx, int64_t ny) { return dim3((unsigned)(nx * ny)); }

// Kernel parameter block shared by the forward kernels (plain values; strides in elements).
struct FwdK {
  int64_t Bsz, D, L, N, G;
  int64_t su[3], sdl[3], sz[3], so[3], soz[3];
  int64_t sA[2], sD, sbias;
  int64_t sB[4], sC[4];  // B/C strides; sB[2] (n) == 1 for the scalar path
  const void* u; const void* delta; const void* z;
  const float* A; const float* Dp; const float* bias;
  const void* Bm; const void* Cm;
  const int32_t* cu; int32_t nseq;
  void* out; void* out_z;
  float* x_ckpt; int64_t nck;   // [Bsz, nck, D, N]: states contiguous, element strides
  int64_t sck[3];               // of the batch, checkpoint and dim axes
  float* last_state;
  float* ws_h;    // [Bsz*D, K, N]  chunk summaries, then carried-in states
  float* ws_s;    // [Bsz*D, K]     sum of Delta since the last sequence start in the chunk
  int32_t* ws_r;  // [Bsz*D, K]     1 if a sequence starts inside the chunk (varlen only)
  int64_t K, Lc;  // number of chunks and chunk length (multiple of kCk)
  int32_t has_D, has_z, has_bias, softplus;
  int64_t nDblk;  // channel blocks per batch: G * ceil(D / G / 64) (chunked kernels) or
                  // G * ceil(D / G / channels per workgroup) (single-pass kernel)
  int32_t nsg;    // dstate > 32: groups of 16 states, one wave each per workgroup (<= 4)
  int32_t lanes;  // 1: single-pass kernel, one lane per (channel, state) (s6_fwd_lanes.hip)
  int32_t rowvec; // 1: chunked kernels read and write whole 8-step row blocks (Row8)
};

}  // namespace s6
