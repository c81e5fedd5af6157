// Causal depthwise conv1d (width 2..4, optional SiLU): the short convolution of the fused
// Mamba path, replacing causal_conv1d_cuda.causal_conv1d_fwd / _bwd
// (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/selective_scan_interface.py:187-189,
// 299-301).
//
// Work layout.  A lane owns VEC adjacent channels (VEC = 8 for 16-bit, 4 for fp32: one
// 16-byte load per lane and step on channel-last storage; VEC = 1 for any other strides)
// and a tile of T consecutive steps; a 256-thread block holds four waves on four adjacent
// tiles of the same 64*VEC channels, so the W-1 halo rows a wave re-reads were just read by
// its neighbour.  Both kernels stream their tensors once and are HBM-bound.
//
// Forward: the last W inputs of each channel sit in a register window that shifts by one
// per step.  Backward: dpre_t = dout_t * act'(pre_t) with pre_t recomputed from x; dx_s =
// sum_k w_k dpre_{s+W-1-k} is accumulated in a second W-deep window and written when its last
// term (t = s+W-1) arrives, so a tile of T outputs walks T+W-1 steps.  dweight / dbias are
// summed per lane over the block's own steps, combined across the block's four waves in
// LDS, written as one partial row per block, and reduced in fixed order by conv_reduce
// (deterministic, no atomics).
#include "s6_internal.h"

namespace s6 {
namespace {

constexpr int kConvWaves = 4;
constexpr int kConvThreads = kConvWaves * kWave;
constexpr int kConvU = 8;     // forward: steps whose loads are issued together
constexpr int kConvUBwd = 4;  // backward (two input streams)

// VEC adjacent elements at p (16-byte aligned when VEC > 1) to / from fp32.
template <typename T, int VEC> struct VIO;
template <typename T> struct VIO<T, 1> {
  __device__ static inline void load(const char* p, float (&f)[1]) { f[0] = Elem<T>::load(p, 0); }
  __device__ static inline void store(char* p, const float (&f)[1]) { Elem<T>::store(p, 0, f[0]); }
};
template <> struct VIO<float, 4> {
  __device__ static inline void load(const char* p, float (&f)[4]) {
    const float4 r = *reinterpret_cast<const float4*>(p);
    f[0] = r.x; f[1] = r.y; f[2] = r.z; f[3] = r.w;
  }
  __device__ static inline void store(char* p, const float (&f)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
  }
};
template <> struct VIO<bf16, 8> {
  __device__ static inline void load(const char* p, float (&f)[8]) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ static inline void store(char* p, const float (&f)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f[2 * i]));
      const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f[2 * i + 1]));
      w[i] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct VIO<f16, 8> {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  __device__ static inline void load(const char* p, float (&f)[8]) {
    const h8 r = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)r[i];
  }
  __device__ static inline void store(char* p, const float (&f)[8]) {
    h8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)f[i];
    *reinterpret_cast<h8*>(p) = r;
  }
};

template <typename T, int VEC>
__device__ inline void zero(float (&f)[VEC]) {
#pragma unroll
  for (int v = 0; v < VEC; ++v) f[v] = 0.f;
}

// Lane geometry shared by both kernels.
struct ConvLane {
  int lane, wv;
  int64_t b, cb, c, cc;  // c: first channel of the lane; cc: c clamped into range
  bool active;
};

template <int VEC>
__device__ inline ConvLane conv_lane(const ConvK& k) {
  ConvLane g;
  g.lane = threadIdx.x & (kWave - 1);
  g.wv = threadIdx.x / kWave;
  g.cb = blockIdx.x % k.nCb;
  g.b = blockIdx.x / k.nCb;
  g.c = (g.cb * kWave + g.lane) * VEC;
  g.active = g.c < k.D;  // VEC > 1 only when D % VEC == 0
  g.cc = g.active ? g.c : 0;
  return g;
}

template <int W, int VEC>
__device__ inline void conv_params(const ConvK& k, int64_t cc, float (&wt)[W][VEC], float (&bs)[VEC]) {
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
#pragma unroll
    for (int j = 0; j < W; ++j) wt[j][v] = k.w[(cc + v) * k.sw[0] + j * k.sw[1]];
    bs[v] = k.bias ? k.bias[(cc + v) * k.sb] : 0.f;
  }
}

// x at steps t0-W+1 .. t0-1 (zero before the sequence start) into win[0 .. W-2].
template <typename T, int W, int VEC>
__device__ inline void load_halo(const char* xp, int64_t xs, int64_t t0, float (&win)[W][VEC]) {
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const int64_t t = t0 - (W - 1) + j;
    if (t >= 0) VIO<T, VEC>::load(xp + t * xs, win[j]);
    else zero<T, VEC>(win[j]);
  }
}

template <typename T, int W, int VEC, bool SILU>
__global__ void __launch_bounds__(kConvThreads) conv_fwd(ConvK k) {
  constexpr int ES = Elem<T>::kSize;
  constexpr int U = kConvU;
  const ConvLane g = conv_lane<VEC>(k);
  const int64_t t0 = ((int64_t)blockIdx.y * kConvWaves + g.wv) * k.T;
  if (t0 >= k.L) return;  // whole wave
  const int64_t t1 = min(t0 + k.T, k.L);
  float wt[W][VEC], bs[VEC];
  conv_params<W, VEC>(k, g.cc, wt, bs);
  const char* const xp = (const char*)k.x + (g.b * k.sx[0] + g.cc * k.sx[1]) * ES;
  char* const op = (char*)k.out + (g.b * k.so[0] + g.cc * k.so[1]) * ES;
  const int64_t xs = k.sx[2] * ES, os = k.so[2] * ES;
  float win[W][VEC];
  load_halo<T, W, VEC>(xp, xs, t0, win);
  for (int64_t tt = t0; tt < t1; tt += U) {
    const int lim = (int)min((int64_t)U, t1 - tt) - 1;
    const char* const xg = xp + tt * xs;
    float cur[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) VIO<T, VEC>::load(xg + min(u, lim) * xs, cur[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) win[W - 1][v] = cur[u][v];
      float o[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        float a = bs[v];
#pragma unroll
        for (int j = 0; j < W; ++j) a = fmaf(wt[j][v], win[j][v], a);
        o[v] = SILU ? a * sigmoidf_(a) : a;
      }
      if (g.active && u <= lim) VIO<T, VEC>::store(op + (tt + u) * os, o);
#pragma unroll
      for (int j = 0; j < W - 1; ++j)
#pragma unroll
        for (int v = 0; v < VEC; ++v) win[j][v] = win[j + 1][v];
    }
  }
}

template <typename T, int W, int VEC, bool SILU>
__global__ void __launch_bounds__(kConvThreads) conv_bwd(ConvK k) {
  constexpr int ES = Elem<T>::kSize;
  constexpr int U = kConvUBwd;
  constexpr int NV = (W + 1) * VEC;  // partial sums per lane: dweight[W][VEC], dbias[VEC]
  __shared__ float red[kConvWaves - 1][NV][kWave];
  const ConvLane g = conv_lane<VEC>(k);
  float wt[W][VEC], bs[VEC];
  conv_params<W, VEC>(k, g.cc, wt, bs);
  const char* const xp = (const char*)k.x + (g.b * k.sx[0] + g.cc * k.sx[1]) * ES;
  const char* const gp = (const char*)k.dout + (g.b * k.sdo[0] + g.cc * k.sdo[1]) * ES;
  char* const dxp = (char*)k.dx + (g.b * k.sdx[0] + g.cc * k.sdx[1]) * ES;
  const int64_t xs = k.sx[2] * ES, gs = k.sdo[2] * ES, dxs = k.sdx[2] * ES;
  float dw[W][VEC], db[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    db[v] = 0.f;
#pragma unroll
    for (int j = 0; j < W; ++j) dw[j][v] = 0.f;
  }
  const int64_t tb0 = (int64_t)blockIdx.y * k.tps;
  const int64_t tb1 = min(tb0 + k.tps, k.ntile4);
  for (int64_t tb = tb0; tb < tb1; ++tb) {
    const int64_t t0 = (tb * kConvWaves + g.wv) * k.T;
    if (t0 >= k.L) continue;  // whole wave
    const int64_t t1 = min(t0 + k.T, k.L);       // steps whose dx this tile writes
    const int64_t te = min(t1 + W - 1, k.L);     // steps whose dpre reach them
    float win[W][VEC], acc[W][VEC];
    load_halo<T, W, VEC>(xp, xs, t0, win);
#pragma unroll
    for (int j = 0; j < W; ++j) zero<T, VEC>(acc[j]);
    for (int64_t tt = t0; tt < te; tt += U) {
      const int lim = (int)min((int64_t)U, te - tt) - 1;
      float xc[U][VEC], gc[U][VEC];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        VIO<T, VEC>::load(xp + (tt + min(u, lim)) * xs, xc[u]);
        VIO<T, VEC>::load(gp + (tt + min(u, lim)) * gs, gc[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u > lim) break;  // uniform
        const int64_t t = tt + u;
        const bool own = t < t1;
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          win[W - 1][v] = xc[u][v];
          float a = bs[v];
#pragma unroll
          for (int j = 0; j < W; ++j) a = fmaf(wt[j][v], win[j][v], a);
          float dp = gc[u][v];
          if (SILU) {  // d silu(a) / da = sig (1 + a (1 - sig))
            const float sg = sigmoidf_(a);
            dp *= sg * fmaf(a, 1.f - sg, 1.f);
          }
          if (own) {
#pragma unroll
            for (int j = 0; j < W; ++j) dw[j][v] = fmaf(dp, win[j][v], dw[j][v]);
            db[v] += dp;
          }
#pragma unroll
          for (int j = 0; j < W; ++j) acc[j][v] = fmaf(wt[j][v], dp, acc[j][v]);
        }
        // acc[0] is dx at s = t - (W - 1), now complete.
        const int64_t s = t - (W - 1);
        if (g.active && s >= t0) VIO<T, VEC>::store(dxp + s * dxs, acc[0]);
#pragma unroll
        for (int j = 0; j < W - 1; ++j)
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            acc[j][v] = acc[j + 1][v];
            win[j][v] = win[j + 1][v];
          }
        zero<T, VEC>(acc[W - 1]);
      }
    }
    // Pending dx for s = te - (W-1) + j: complete only where te is the sequence end.
#pragma unroll
    for (int j = 0; j < W - 1; ++j) {
      const int64_t s = te - (W - 1) + j;
      if (g.active && s >= t0 && s < t1) VIO<T, VEC>::store(dxp + s * dxs, acc[j]);
    }
  }
  // Block sum of the four waves' partials; wave 0 writes the block's row.
  if (g.wv > 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
#pragma unroll
      for (int j = 0; j < W; ++j) red[g.wv - 1][j * VEC + v][g.lane] = dw[j][v];
      red[g.wv - 1][W * VEC + v][g.lane] = db[v];
    }
  }
  __syncthreads();
  if (g.wv == 0 && g.active) {
    float* const row = k.ws + ((g.b * k.nsplit + blockIdx.y) * k.D + g.c) * (W + 1);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
#pragma unroll
      for (int j = 0; j <= W; ++j) {
        float s = j < W ? dw[j][v] : db[v];
#pragma unroll
        for (int w = 0; w < kConvWaves - 1; ++w) s += red[w][j * VEC + v][g.lane];
        row[v * (W + 1) + j] = s;
      }
    }
  }
}

// dweight[d, j] (j < W) and dbias[d] (j == W) as the sum over the Bsz * nsplit partial rows,
// in row order.  One thread per (d, j).
template <int W>
__global__ void __launch_bounds__(256) conv_reduce(ConvK k) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = k.D * (W + 1);
  if (i >= n) return;
  const int64_t rows = k.Bsz * k.nsplit;
  float s = 0.f;
  for (int64_t r = 0; r < rows; ++r) s += k.ws[r * n + i];
  const int64_t d = i / (W + 1);
  const int j = (int)(i % (W + 1));
  if (j < W) k.dw[d * k.sdw[0] + j * k.sdw[1]] = s;
  else if (k.dbias) k.dbias[d * k.sdb] = s;
}

template <typename T, int W, int VEC, bool SILU>
hipError_t conv_fwd_t(const ConvK& k, hipStream_t st) {
  const dim3 grid((unsigned)(k.nCb * k.Bsz), (unsigned)k.ntile4);
  hipLaunchKernelGGL((conv_fwd<T, W, VEC, SILU>), grid, dim3(kConvThreads), 0, st, k);
  return hipGetLastError();
}

template <typename T, int W, int VEC, bool SILU>
hipError_t conv_bwd_t(const ConvK& k, hipStream_t st) {
  const dim3 grid((unsigned)(k.nCb * k.Bsz), (unsigned)k.nsplit);
  hipLaunchKernelGGL((conv_bwd<T, W, VEC, SILU>), grid, dim3(kConvThreads), 0, st, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t n = k.D * (W + 1);
  hipLaunchKernelGGL((conv_reduce<W>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, k);
  return hipGetLastError();
}

template <bool BWD, typename T, int VEC>
hipError_t conv_dispatch_w(const ConvK& k, int width, bool silu, hipStream_t st) {
#define S6_CONV_CASE(W_)                                                              \
  case W_:                                                                            \
    if (BWD) return silu ? conv_bwd_t<T, W_, VEC, true>(k, st) : conv_bwd_t<T, W_, VEC, false>(k, st); \
    return silu ? conv_fwd_t<T, W_, VEC, true>(k, st) : conv_fwd_t<T, W_, VEC, false>(k, st);
  switch (width) {
    S6_CONV_CASE(2)
    S6_CONV_CASE(3)
    S6_CONV_CASE(4)
    default: return hipErrorInvalidValue;
  }
#undef S6_CONV_CASE
}

template <bool BWD>
hipError_t conv_dispatch(const ConvK& k, int io_dtype, int width, int vec, bool silu, hipStream_t st) {
  switch (io_dtype) {
    case S6_F32:
      return vec == 4 ? conv_dispatch_w<BWD, float, 4>(k, width, silu, st)
                      : conv_dispatch_w<BWD, float, 1>(k, width, silu, st);
    case S6_BF16:
      return vec == 8 ? conv_dispatch_w<BWD, bf16, 8>(k, width, silu, st)
                      : conv_dispatch_w<BWD, bf16, 1>(k, width, silu, st);
    case S6_F16:
      return vec == 8 ? conv_dispatch_w<BWD, f16, 8>(k, width, silu, st)
                      : conv_dispatch_w<BWD, f16, 1>(k, width, silu, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_conv_fwd(const ConvK& k, int io_dtype, int width, int vec, bool silu,
                           hipStream_t st) {
  return conv_dispatch<false>(k, io_dtype, width, vec, silu, st);
}

hipError_t launch_conv_bwd(const ConvK& k, int io_dtype, int width, int vec, bool silu,
                           hipStream_t st) {
  return conv_dispatch<true>(k, io_dtype, width, vec, silu, st);
}

}  // namespace s6
