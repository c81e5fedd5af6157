// Causal depthwise conv1d (width 2..4, optional SiLU): the short convolution of the fused
// Mamba path, replacing causal_conv1d_cuda.causal_conv1d_fwd / _bwd
// (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/selective_scan_interface.py:187-189,
// 299-301).
//
// Work layout.  A lane owns VEC adjacent channels (VEC in 8 / 4 / 2 for channel-last
// storage, chosen by the host so that few lanes idle: one 4- to 16-byte load per lane and
// step; VEC = 1 for any other strides) and a tile of T consecutive steps; a 256-thread block holds four waves on four adjacent
// tiles of the same 64*VEC channels, so the W-1 halo rows a wave re-reads were just read by
// its neighbour.  Both kernels stream their tensors once and are HBM-bound.
//
// Forward: the last W inputs of each channel sit in a register window that shifts by one
// per step.  Backward: dpre_t = dout_t * act'(pre_t) with pre_t recomputed from x; dx_s =
// sum_k w_k dpre_{s+W-1-k} is accumulated in a second W-deep window and written when its last
// term (t = s+W-1) arrives, so a tile of T outputs walks T+W-1 steps.  dweight / dbias are
// summed per lane over the block's own steps, combined across the block's four waves in
// LDS, written as one partial row per block, and reduced in fixed order by two conv_colsum
// launches (deterministic, no atomics).
#include "s6_internal.h"

namespace s6 {
namespace {

constexpr int kConvWaves = 4;

// 1 / (1 + e^-x) with the hardware exp2 on the rounded product -x log2(e): relative error
// below |x| 6e-8 + 2 ulp, well inside fp32 parity for the activation's range.
__device__ inline float conv_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
constexpr int kConvThreads = kConvWaves * kWave;
constexpr int kConvU = 8;     // forward: steps per load group (one group in flight ahead)
constexpr int kConvUBwd = 4;  // backward (two input streams)

// VEC adjacent elements at p (aligned to their total size) to / from fp32.  load_raw
// fetches the packed bits (Raw) so that a group of loads can be in flight while the previous
// group is computed; unpack converts them when they are used.
template <int BYTES> struct RawOf;
template <> struct RawOf<2> { typedef uint16_t type; };
template <> struct RawOf<4> { typedef uint32_t type; };
template <> struct RawOf<8> { typedef uint2 type; };
template <> struct RawOf<16> { typedef uint4 type; };

template <int NW>
__device__ inline void words(const typename RawOf<NW * 4>::type& r, uint32_t (&w)[NW]);
template <> __device__ inline void words<1>(const uint32_t& r, uint32_t (&w)[1]) { w[0] = r; }
template <> __device__ inline void words<2>(const uint2& r, uint32_t (&w)[2]) { w[0] = r.x; w[1] = r.y; }
template <> __device__ inline void words<4>(const uint4& r, uint32_t (&w)[4]) {
  w[0] = r.x; w[1] = r.y; w[2] = r.z; w[3] = r.w;
}
template <int NW>
__device__ inline typename RawOf<NW * 4>::type pack_words(const uint32_t (&w)[NW]);
template <> __device__ inline uint32_t pack_words<1>(const uint32_t (&w)[1]) { return w[0]; }
template <> __device__ inline uint2 pack_words<2>(const uint32_t (&w)[2]) { return make_uint2(w[0], w[1]); }
template <> __device__ inline uint4 pack_words<4>(const uint32_t (&w)[4]) {
  return make_uint4(w[0], w[1], w[2], w[3]);
}

template <typename T> __device__ inline float from_bits(uint32_t h);
template <> __device__ inline float from_bits<bf16>(uint32_t h) { return __uint_as_float(h << 16); }
template <> __device__ inline float from_bits<f16>(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
template <typename T> __device__ inline uint32_t to_bits(float v);
template <> __device__ inline uint32_t to_bits<bf16>(float v) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}
template <> __device__ inline uint32_t to_bits<f16>(float v) {
  asm("" : "+v"(v));  // rounded to fp32 first (see Buf<f16>::store)
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

template <typename T, int VEC> struct VIO {
  static constexpr int ES = Elem<T>::kSize;
  static constexpr int BYTES = ES * VEC;
  typedef typename RawOf<BYTES>::type Raw;
  __device__ static inline Raw load_raw(const char* p) { return *reinterpret_cast<const Raw*>(p); }
  __device__ static inline void unpack(const Raw& r, float (&f)[VEC]) {
    if constexpr (ES == 4) {
      uint32_t w[VEC];
      words<VEC>(r, w);
#pragma unroll
      for (int v = 0; v < VEC; ++v) f[v] = __uint_as_float(w[v]);
    } else if constexpr (VEC == 1) {
      f[0] = from_bits<T>((uint32_t)r);
    } else {
      uint32_t w[VEC / 2];
      words<VEC / 2>(r, w);
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i) {
        f[2 * i] = from_bits<T>(w[i] & 0xffffu);
        f[2 * i + 1] = from_bits<T>(w[i] >> 16);
      }
    }
  }
  __device__ static inline void load(const char* p, float (&f)[VEC]) { unpack(load_raw(p), f); }
  __device__ static inline void store(char* p, const float (&f)[VEC]) {
    Raw r;
    if constexpr (ES == 4) {
      uint32_t w[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) w[v] = __float_as_uint(f[v]);
      r = pack_words<VEC>(w);
    } else if constexpr (VEC == 1) {
      r = (uint16_t)to_bits<T>(f[0]);
    } else {
      uint32_t w[VEC / 2];
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i) w[i] = to_bits<T>(f[2 * i]) | (to_bits<T>(f[2 * i + 1]) << 16);
      r = pack_words<VEC / 2>(w);
    }
    *reinterpret_cast<Raw*>(p) = r;
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
  // Group g + 1's loads are issued before group g is computed.
  typedef typename VIO<T, VEC>::Raw Raw;
  Raw nx[U];
  auto issue = [&](int64_t base) {
    const int lim = (int)min((int64_t)U, t1 - base) - 1;
#pragma unroll
    for (int u = 0; u < U; ++u) nx[u] = VIO<T, VEC>::load_raw(xp + (base + min(u, lim)) * xs);
  };
  issue(t0);
  for (int64_t tt = t0; tt < t1; tt += U) {
    const int lim = (int)min((int64_t)U, t1 - tt) - 1;
    Raw cx[U];
#pragma unroll
    for (int u = 0; u < U; ++u) cx[u] = nx[u];
    if (tt + U < t1) issue(tt + U);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      VIO<T, VEC>::unpack(cx[u], win[W - 1]);
      float o[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        float a = bs[v];
#pragma unroll
        for (int j = 0; j < W; ++j) a = fmaf(wt[j][v], win[j][v], a);
        o[v] = SILU ? a * conv_sigmoid(a) : a;
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
    typedef typename VIO<T, VEC>::Raw Raw;
    Raw nx[U], ng[U];
    auto issue = [&](int64_t base) {
      const int lim = (int)min((int64_t)U, te - base) - 1;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        nx[u] = VIO<T, VEC>::load_raw(xp + (base + min(u, lim)) * xs);
        ng[u] = VIO<T, VEC>::load_raw(gp + (base + min(u, lim)) * gs);
      }
    };
    issue(t0);
    for (int64_t tt = t0; tt < te; tt += U) {
      const int lim = (int)min((int64_t)U, te - tt) - 1;
      Raw cx[U], cg[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        cx[u] = nx[u];
        cg[u] = ng[u];
      }
      if (tt + U < te) issue(tt + U);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u > lim) break;  // uniform
        float gc[VEC];
        VIO<T, VEC>::unpack(cx[u], win[W - 1]);
        VIO<T, VEC>::unpack(cg[u], gc);
        const int64_t t = tt + u;
        const bool own = t < t1;
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          float a = bs[v];
#pragma unroll
          for (int j = 0; j < W; ++j) a = fmaf(wt[j][v], win[j][v], a);
          float dp = gc[v];
          if (SILU) {  // d silu(a) / da = sig (1 + a (1 - sig))
            const float sg = conv_sigmoid(a);
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

// Column sums of the [R, n] partial matrix (n = D * (W + 1)) in two fixed-order levels:
// block (x, y) sums rows [y * rps, min((y + 1) * rps, R)) of columns [64 x, 64 x + 64), the
// four waves taking every fourth row and combining in LDS; the first level writes one row
// per slice to ws2, the second (one slice) sums those rows into dweight[d, j] (j < W) and
// dbias[d] (j == W).
template <int W, bool FINAL>
__global__ void __launch_bounds__(kConvThreads) conv_colsum(ConvK k, const float* src, int64_t R,
                                                            int64_t rps, float* dst) {
  __shared__ float red[kConvWaves - 1][kWave];
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const int64_t n = k.D * (W + 1);
  const int64_t col = (int64_t)blockIdx.x * kWave + lane;
  const int64_t r0 = (int64_t)blockIdx.y * rps, r1 = min(r0 + rps, R);
  float s = 0.f;
  if (col < n) {
#pragma unroll 8
    for (int64_t r = r0 + wv; r < r1; r += kConvWaves) s += src[r * n + col];
  }
  if (wv > 0) red[wv - 1][lane] = s;
  __syncthreads();
  if (wv != 0 || col >= n) return;
#pragma unroll
  for (int w = 0; w < kConvWaves - 1; ++w) s += red[w][lane];
  if (!FINAL) {
    dst[blockIdx.y * n + col] = s;
  } else {
    const int64_t d = col / (W + 1);
    const int j = (int)(col % (W + 1));
    if (j < W) k.dw[d * k.sdw[0] + j * k.sdw[1]] = s;
    else if (k.dbias) k.dbias[d * k.sdb] = s;
  }
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
  const unsigned nx = (unsigned)((k.D * (W + 1) + kWave - 1) / kWave);
  const int64_t R = k.Bsz * k.nsplit;
  hipLaunchKernelGGL((conv_colsum<W, false>), dim3(nx, (unsigned)k.nslice), dim3(kConvThreads), 0,
                     st, k, (const float*)k.ws, R, k.rps, k.ws2);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((conv_colsum<W, true>), dim3(nx, 1u), dim3(kConvThreads), 0, st, k,
                     (const float*)k.ws2, k.nslice, k.nslice, (float*)nullptr);
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
      switch (vec) {
        case 4: return conv_dispatch_w<BWD, float, 4>(k, width, silu, st);
        case 2: return conv_dispatch_w<BWD, float, 2>(k, width, silu, st);
        case 1: return conv_dispatch_w<BWD, float, 1>(k, width, silu, st);
      }
      break;
    case S6_BF16:
      switch (vec) {
        case 8: if constexpr (!BWD) return conv_dispatch_w<BWD, bf16, 8>(k, width, silu, st); break;
        case 4: return conv_dispatch_w<BWD, bf16, 4>(k, width, silu, st);
        case 2: return conv_dispatch_w<BWD, bf16, 2>(k, width, silu, st);
        case 1: return conv_dispatch_w<BWD, bf16, 1>(k, width, silu, st);
      }
      break;
    case S6_F16:
      switch (vec) {
        case 8: if constexpr (!BWD) return conv_dispatch_w<BWD, f16, 8>(k, width, silu, st); break;
        case 4: return conv_dispatch_w<BWD, f16, 4>(k, width, silu, st);
        case 2: return conv_dispatch_w<BWD, f16, 2>(k, width, silu, st);
        case 1: return conv_dispatch_w<BWD, f16, 1>(k, width, silu, st);
      }
      break;
  }
  return hipErrorInvalidValue;
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
