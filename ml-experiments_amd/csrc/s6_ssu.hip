// selective_state_update: one recurrent decode step of the S6 state, in place
// (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/selective_state_update.py:
// 18-118 kernel, 204-265 reference semantics).
//
// Two mappings.  Rows with contiguous, aligned states and dstate a power of two in [4, 256]
// (the usual case): dstate / 4 lanes per row, 4 states per lane, so every load of the
// state and A is one contiguous 16-byte piece per lane and a wave reads whole rows.  Any
// other layout: one lane per (batch, head, channel) row, 256 rows per workgroup, walking the row's
// states in groups of 16 whose loads (state, A, B, C) are all issued before the group is
// computed.  B / C rows are the same for every lane of a wave
// (one (batch, group) per wave), so their loads are broadcasts from one cache line.  The
// step is latency-bound at decode sizes: state bytes read + written per call (e.g. 12.6 MB
// for batch 64, dim 1536, dstate 16 in fp32) are a few microseconds at HBM rate.
#include "s6_internal.h"
#include "selective_state_update.h"

namespace s6 {
namespace {

// The state's storage type is a template parameter; the row tensors' and B / C's dtypes are
// wave-uniform runtime switches (load_any / store_any, one or two elements per lane).

constexpr int kSsuGroup = 16;

// Four waves per workgroup: the step launches few, short waves, so the workgroup dispatch
// rate, not HBM, bounds one-wave workgroups at large batch.
constexpr int kSsuThreads = 4 * kWave;

template <typename Ts, bool SOFTPLUS>
__global__ void __launch_bounds__(kSsuThreads) ssu_kernel(SsuK k) {
  const int64_t d = (int64_t)blockIdx.x * kSsuThreads + threadIdx.x;
  if (d >= k.dim) return;  // no barriers below
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t g = h / k.hpg;
  const float x = load_any(k.x, b * k.sx[0] + h * k.sx[1] + d * k.sx[2], k.io);
  float dt = load_any(k.dt, b * k.sdt[0] + h * k.sdt[1] + d * k.sdt[2], k.io);
  if (k.bias) dt += k.bias[h * k.sbias[0] + d * k.sbias[1]];
  if (SOFTPLUS) dt = softplus20(dt);
  const int64_t st = b * k.ss[0] + h * k.ss[1] + d * k.ss[2];
  const int64_t ar = h * k.sA[0] + d * k.sA[1];
  const int64_t br = b * k.sB[0] + g * k.sB[1];
  const int64_t cr = b * k.sC[0] + g * k.sC[1];
  const int64_t N = k.dstate;
  float acc = 0.f;
  for (int64_t n0 = 0; n0 < N; n0 += kSsuGroup) {
    float s[kSsuGroup], a[kSsuGroup], bb[kSsuGroup], cc[kSsuGroup];
#pragma unroll
    for (int j = 0; j < kSsuGroup; ++j) {
      const int64_t n = min(n0 + j, N - 1);  // in range; the tail is not stored
      s[j] = Elem<Ts>::load(k.state, st + n * k.ss[3]);
      a[j] = k.A[ar + n * k.sA[2]];
      bb[j] = load_any(k.B, br + n * k.sB[2], k.bc);
      cc[j] = load_any(k.C, cr + n * k.sC[2], k.bc);
    }
#pragma unroll
    for (int j = 0; j < kSsuGroup; ++j) {
      if (n0 + j < N) {
        // state * exp(A dt) + (B dt) x, the reference's operand order
        const float ns = fmaf(s[j], exp_split(a[j] * dt), (bb[j] * dt) * x);
        Elem<Ts>::store(k.state, st + (n0 + j) * k.ss[3], ns);
        acc = fmaf(ns, cc[j], acc);
      }
    }
  }
  float o = acc;
  if (k.Dp) o = fmaf(x, k.Dp[h * k.sD[0] + d * k.sD[1]], o);
  if (k.z) {
    const float zz = load_any(k.z, b * k.sz[0] + h * k.sz[1] + d * k.sz[2], k.io);
    o *= zz * sigmoidf_(zz);
  }
  store_any(k.out, b * k.so[0] + h * k.so[1] + d * k.so[2], o, k.io);
}

// Rows whose states are contiguous (state stride 1 along dstate, dstate % 4 == 0, rows
// aligned to four elements): LPR lanes share a row, 4 states per lane, so a wave reads whole
// contiguous rows with one load per lane; A and B / C take one vector load each when they
// are contiguous too (a_vec, bc_vec), else four strided loads (A's zero strides of the
// tied-head-dim form included); out is reduced across the row's lanes.  LPR = dstate / 4, a power of two from 1 to 64; other dstate values take the
// lane-per-row kernel above.
template <typename Ts> struct Vec4;
template <> struct Vec4<float> {
  __device__ static inline void load(const void* p, float (&f)[4]) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
  }
  __device__ static inline void store(void* p, const float (&f)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
  }
};
template <typename Ts> struct Vec4 {  // 16-bit storage: 8 bytes
  __device__ static inline void load(const void* p, float (&f)[4]) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      f[2 * i] = Elem<Ts>::load(&w[i], 0);
      f[2 * i + 1] = Elem<Ts>::load(&w[i], 1);
    }
  }
  __device__ static inline void store(void* p, const float (&f)[4]) {
    uint32_t w[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      Elem<Ts>::store(&w[i], 0, f[2 * i]);
      Elem<Ts>::store(&w[i], 1, f[2 * i + 1]);
    }
    *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  }
};

// Four contiguous elements at element offset i (aligned to four elements).
__device__ inline void load4_any(const void* p, int64_t i, int dt, float (&f)[4]) {
  if (dt == S6_F32) Vec4<float>::load((const char*)p + i * 4, f);
  else if (dt == S6_BF16) Vec4<bf16>::load((const char*)p + i * 2, f);
  else Vec4<f16>::load((const char*)p + i * 2, f);
}

template <typename Ts, bool SOFTPLUS, int LPR>
__global__ void __launch_bounds__(kSsuThreads) ssu_rows_kernel(SsuK k) {
  constexpr int RPB = kSsuThreads / LPR;  // rows per workgroup (a row never spans two waves)
  const int sub = threadIdx.x % LPR;
  const int64_t d = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const bool live = d < k.dim;
  const int64_t dd = live ? d : k.dim - 1;  // dead lanes compute a valid row, store nothing
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t g = h / k.hpg;
  // Every load is issued before any arithmetic: one memory round trip per step.
  const int64_t n0 = 4 * sub;
  char* const sp = (char*)k.state + (b * k.ss[0] + h * k.ss[1] + dd * k.ss[2] + n0) * Elem<Ts>::kSize;
  float s[4], a[4], bb[4], cc[4];
  Vec4<Ts>::load(sp, s);
  const int64_t ar = h * k.sA[0] + dd * k.sA[1];
  if (k.a_vec) {
    Vec4<float>::load(k.A + ar + n0, a);
  } else {  // any stride, including the tied-head-dim broadcast (stride 0)
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = k.A[ar + (n0 + j) * k.sA[2]];
  }
  const int64_t br = b * k.sB[0] + g * k.sB[1], cr = b * k.sC[0] + g * k.sC[1];
  if (k.bc_vec) {
    load4_any(k.B, br + n0, k.bc, bb);
    load4_any(k.C, cr + n0, k.bc, cc);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bb[j] = load_any(k.B, br + (n0 + j) * k.sB[2], k.bc);
      cc[j] = load_any(k.C, cr + (n0 + j) * k.sC[2], k.bc);
    }
  }
  const float x = load_any(k.x, b * k.sx[0] + h * k.sx[1] + dd * k.sx[2], k.io);
  float dt = load_any(k.dt, b * k.sdt[0] + h * k.sdt[1] + dd * k.sdt[2], k.io);
  const float bias = k.bias ? k.bias[h * k.sbias[0] + dd * k.sbias[1]] : 0.f;
  const float Dv = k.Dp ? k.Dp[h * k.sD[0] + dd * k.sD[1]] : 0.f;
  const float zz = k.z ? load_any(k.z, b * k.sz[0] + h * k.sz[1] + dd * k.sz[2], k.io) : 0.f;
  dt += bias;
  if (SOFTPLUS) dt = softplus20(dt);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s[j] = fmaf(s[j], exp_split(a[j] * dt), (bb[j] * dt) * x);
    acc = fmaf(s[j], cc[j], acc);
  }
  if (live) Vec4<Ts>::store(sp, s);
#pragma unroll
  for (int m = LPR / 2; m >= 1; m /= 2) acc += __shfl_xor(acc, m, LPR);
  if (!live || sub != 0) return;
  float o = fmaf(x, Dv, acc);
  if (k.z) o *= zz * sigmoidf_(zz);
  store_any(k.out, b * k.so[0] + h * k.so[1] + d * k.so[2], o, k.io);
}

template <typename Ts, bool SP, int LPR>
void ssu_rows_launch(const SsuK& k, hipStream_t st) {
  constexpr int RPB = kSsuThreads / LPR;
  const dim3 grid((unsigned)((k.dim + RPB - 1) / RPB), (unsigned)k.nheads, (unsigned)k.batch);
  hipLaunchKernelGGL((ssu_rows_kernel<Ts, SP, LPR>), grid, dim3(kSsuThreads), 0, st, k);
}

template <typename Ts, bool SP>
bool ssu_rows(const SsuK& k, hipStream_t st) {
  switch (k.dstate) {
    case 4: ssu_rows_launch<Ts, SP, 1>(k, st); return true;
    case 8: ssu_rows_launch<Ts, SP, 2>(k, st); return true;
    case 16: ssu_rows_launch<Ts, SP, 4>(k, st); return true;
    case 32: ssu_rows_launch<Ts, SP, 8>(k, st); return true;
    case 64: ssu_rows_launch<Ts, SP, 16>(k, st); return true;
    case 128: ssu_rows_launch<Ts, SP, 32>(k, st); return true;
    case 256: ssu_rows_launch<Ts, SP, 64>(k, st); return true;
    default: return false;
  }
}

template <typename Ts>
hipError_t ssu_t(const SsuK& k, bool softplus, bool rows, hipStream_t st) {
  if (rows && (softplus ? ssu_rows<Ts, true>(k, st) : ssu_rows<Ts, false>(k, st)))
    return hipGetLastError();
  const dim3 grid((unsigned)((k.dim + kSsuThreads - 1) / kSsuThreads), (unsigned)k.nheads,
                  (unsigned)k.batch);
  if (softplus) hipLaunchKernelGGL((ssu_kernel<Ts, true>), grid, dim3(kSsuThreads), 0, st, k);
  else hipLaunchKernelGGL((ssu_kernel<Ts, false>), grid, dim3(kSsuThreads), 0, st, k);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_state_update(const SsuK& k, int state_dtype, bool softplus, bool rows,
                               hipStream_t st) {
  switch (state_dtype) {
    case S6_F32: return ssu_t<float>(k, softplus, rows, st);
    case S6_BF16: return ssu_t<bf16>(k, softplus, rows, st);
    case S6_F16: return ssu_t<f16>(k, softplus, rows, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace s6
