// Backward S6 selective scan for gfx950.
//
// With lambda_t = dL/dh_t and g_t = abar_t * lambda_t (the gradient that step t passes to
// h_{t-1}):
//     lambda_t = C_t dy_t + g_{t+1},     g_t = abar_t lambda_t   (g_t = 0 at a sequence start)
//     q_t = abar_t h_{t-1} lambda_t   (gradient of the exponent Delta_t A)
//     dA += q Delta,  dDelta = sum_n q A + u sum_n lambda B,  du = Delta sum_n lambda B + D dy
//     dB_t += lambda Delta u,  dC_t += dy h_t        (summed over the channels of a group)
// These are the gradients autograd produces through selective_scan_ref
// (selective_scan_interface.py:107-156); the reference's native bwd is replaced here.
//
// Kernels (the reverse mirror of the forward's chunking):
//   bwd_summary  per chunk c >= 1: g leaving the chunk at its first step, from a zero
//                inflow, and the chunk's sum of Delta.
//   bwd_carry    reverse prefix over chunks: g entering each chunk.
//   bwd_main     per chunk, per 32-step checkpoint interval (in reverse): reload the state
//                saved by the forward, recompute 8-step segments forward into registers,
//                then run the reverse recurrence.  dB/dC are reduced over the 64 lanes of a
//                wave with permlane swaps and DPP, then over the 4 waves of the workgroup in
//                LDS, and written as one partial per 256-channel block (deterministic).
//   bwd_reduce_bc  sums the partials into dB / dC.
#include "s6_internal.h"
#include "s6_wave.h"

namespace s6 {

namespace {

__device__ inline int64_t last_start_le(const int32_t* cu, int32_t nseq, int64_t t) {
  int32_t lo = 0, hi = nseq + 1;  // first i with cu[i] > t
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if ((int64_t)cu[mid] <= t) lo = mid + 1; else hi = mid;
  }
  return (lo > 0) ? (int64_t)cu[lo - 1] : -1;
}

// Bit i set when a sequence starts at step ts + i, for i in [0, te - ts) (te - ts <= 32).
__device__ inline uint32_t start_mask(const int32_t* cu, int32_t nseq, int64_t ts, int64_t te) {
  int32_t lo = 0, hi = nseq + 1;  // first i with cu[i] >= ts
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if ((int64_t)cu[mid] < ts) lo = mid + 1; else hi = mid;
  }
  uint32_t m = 0;
  for (int32_t i = lo; i <= nseq && (int64_t)cu[i] < te; ++i) m |= 1u << (uint32_t)(cu[i] - ts);
  return m;
}

__device__ inline bool chunk_has_start(const int32_t* cu, int32_t nseq, int64_t t0, int64_t t1) {
  int32_t lo = 0, hi = nseq + 1;
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if ((int64_t)cu[mid] < t0) lo = mid + 1; else hi = mid;
  }
  return lo <= nseq && (int64_t)cu[lo] < t1;
}

}  // namespace

template <typename Tio, typename Tbc, int NS, bool VARLEN>
__global__ void __launch_bounds__(kWave) bwd_summary(BwdK p) {
  const int lane = threadIdx.x;
  const int64_t Dg = p.D / p.G;
  const int64_t nJ = (Dg + kWave - 1) / kWave;
  const int64_t blk = blockIdx.x;
  const int64_t b = blk / p.nDblk;
  const int64_t rem = blk % p.nDblk;
  const int64_t g = rem / nJ;
  const int64_t j = rem % nJ;
  const int64_t dloc = j * kWave + lane;
  const bool active = dloc < Dg;
  const int64_t d = g * Dg + (active ? dloc : Dg - 1);
  const int64_t c = blockIdx.y + 1;
  const int64_t t0 = c * p.Lc;
  const int64_t t1 = min(t0 + p.Lc, p.L);
  const int N = (int)p.N;
  const int64_t ch = b * p.D + d;

  float Ap[NS], gs[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    Ap[n] = (n < N) ? p.A[d * p.sA[0] + n * p.sA[1]] * kLog2e : 0.f;
    gs[n] = 0.f;
  }
  const float bias = p.has_bias ? p.bias[d * p.sbias] : 0.f;
  const int64_t ub = b * p.sdl[0] + d * p.sdl[1];
  const int64_t zb = b * p.sz[0] + d * p.sz[1];
  const int64_t dob = b * p.sdo[0] + d * p.sdo[1];
  const char* Cbase = (const char*)p.Cm + (b * p.sC[0] + g * p.sC[1]) * Elem<Tbc>::kSize;
  const int64_t Cstep = p.sC[3] * Elem<Tbc>::kSize;
  int64_t ps = VARLEN ? last_start_le(p.cu, p.nseq, t1 - 1) : -1;
  float ssum = 0.f;
  for (int64_t t = t1 - 1; t >= t0; --t) {
    float Cv[NS];
    BCLoad<Tbc>::template row<NS>(Cbase + t * Cstep, Cv);
    float dy = Elem<Tio>::load(p.dout, dob + t * p.sdo[2]);
    if (p.has_z) {
      const float zz = Elem<Tio>::load(p.z, zb + t * p.sz[2]);
      dy *= zz * sigmoidf_(zz);
    }
    float dt = Elem<Tio>::load(p.delta, ub + t * p.sdl[2]) + bias;
    if (p.softplus) dt = softplus20(dt);
    const bool st = VARLEN && t == ps;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const float lam = fmaf(Cv[n], dy, gs[n]);
      const float a = fast_exp2(dt * Ap[n]);
      gs[n] = st ? 0.f : a * lam;
    }
    ssum += dt;
    if (st) ps = last_start_le(p.cu, p.nseq, t - 1);
  }
  if (active) {
    float* go = p.ws_g + (ch * p.K + c) * p.N;
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) go[n] = gs[n];
    p.ws_s[ch * p.K + c] = ssum;
  }
}

__global__ void __launch_bounds__(256) bwd_carry(BwdK p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = p.Bsz * p.D * p.N;
  if (i >= total) return;
  const int64_t ch = i / p.N;
  const int64_t n = i % p.N;
  const int64_t d = ch % p.D;
  const float ap = p.A[d * p.sA[0] + n * p.sA[1]] * kLog2e;
  float gin = 0.f;
  for (int64_t c = p.K - 1; c >= 0; --c) {
    float* slot = p.ws_g + (ch * p.K + c) * p.N + n;
    const float gloc = (c >= 1) ? *slot : 0.f;
    *slot = gin;
    if (c >= 1) {
      const int64_t t0 = c * p.Lc, t1 = min(t0 + p.Lc, p.L);
      const bool reset = p.nseq > 0 && chunk_has_start(p.cu, p.nseq, t0, t1);
      const float decay = fast_exp2(ap * p.ws_s[ch * p.K + c]);
      gin = (reset ? 0.f : decay * gin) + gloc;
    }
  }
}

template <typename Tio, typename Tbc, bool VARLEN>
__global__ void __launch_bounds__(256) bwd_main(BwdK p) {
  constexpr int NS = 16;
  constexpr int SEG = 8;
  constexpr int NSEG = kCk / SEG;
  __shared__ float s_seg[NSEG][NS][256];   // state at the start of each segment
  __shared__ float s_red[2][SEG][4][NS];   // per-wave dB / dC sums for one segment

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int64_t Dg = p.D / p.G;
  const int64_t blk = blockIdx.x;
  const int64_t b = blk / (p.G * p.nJ4);
  const int64_t rem = blk % (p.G * p.nJ4);
  const int64_t g = rem / p.nJ4;
  const int64_t j4 = rem % p.nJ4;
  const int64_t dloc = j4 * 256 + tid;
  const bool active = dloc < Dg;
  const int64_t d = g * Dg + (active ? dloc : Dg - 1);
  const int64_t c = blockIdx.y;
  const int64_t t0 = c * p.Lc;
  const int64_t t1 = min(t0 + p.Lc, p.L);
  const int N = (int)p.N;
  const int64_t ch = b * p.D + d;

  float Ap[NS], gs[NS], dAacc[NS];
  {
    const float* gin = p.ws_g + (ch * p.K + c) * p.N;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      Ap[n] = (n < N) ? p.A[d * p.sA[0] + n * p.sA[1]] * kLog2e : 0.f;
      gs[n] = (n < N && p.K > 1) ? gin[n] : 0.f;
      dAacc[n] = 0.f;
    }
  }
  const float bias = p.has_bias ? p.bias[d * p.sbias] : 0.f;
  const float Dv = p.has_D ? p.Dp[d * p.sD] : 0.f;
  float dDacc = 0.f, dbacc = 0.f;

  const int64_t ub = b * p.su[0] + d * p.su[1];
  const int64_t db = b * p.sdl[0] + d * p.sdl[1];
  const int64_t zb = b * p.sz[0] + d * p.sz[1];
  const int64_t dob = b * p.sdo[0] + d * p.sdo[1];
  const int64_t oub = b * p.sout[0] + d * p.sout[1];
  const int64_t dub = b * p.sdu[0] + d * p.sdu[1];
  const int64_t ddb = b * p.sddl[0] + d * p.sddl[1];
  const int64_t dzb = b * p.sdz[0] + d * p.sdz[1];
  const char* Bbase = (const char*)p.Bm + (b * p.sB[0] + g * p.sB[1]) * Elem<Tbc>::kSize;
  const char* Cbase = (const char*)p.Cm + (b * p.sC[0] + g * p.sC[1]) * Elem<Tbc>::kSize;
  const int64_t Bstep = p.sB[3] * Elem<Tbc>::kSize;
  const int64_t Cstep = p.sC[3] * Elem<Tbc>::kSize;
  float* pBrow = p.ws_pB + ((b * p.G + g) * p.nJ4 + j4) * p.L * p.N;
  float* pCrow = p.ws_pC + ((b * p.G + g) * p.nJ4 + j4) * p.L * p.N;

  const int64_t nsub = (t1 - t0 + kCk - 1) / kCk;
  for (int64_t s = nsub - 1; s >= 0; --s) {
    const int64_t ts = t0 + s * kCk;
    const int64_t te = min(ts + kCk, t1);
    const uint32_t smask = VARLEN ? start_mask(p.cu, p.nseq, ts, te) : 0u;
    float h[NS];
    if (ts == 0) {
#pragma unroll
      for (int n = 0; n < NS; ++n) h[n] = 0.f;
    } else {
      const float* xc = p.x_ckpt + (ch * p.nck + ts / kCk - 1) * p.N;
#pragma unroll
      for (int n = 0; n < NS; ++n) h[n] = (n < N) ? xc[n] : 0.f;
    }
    // Pre-pass: states at the segment starts.
    for (int k = 0; k < NSEG; ++k) {
#pragma unroll
      for (int n = 0; n < NS; ++n) s_seg[k][n][tid] = h[n];
      const int64_t sg0 = ts + k * SEG;
#pragma unroll
      for (int i = 0; i < SEG; ++i) {
        const int64_t t = sg0 + i;
        if (t < te) {
          if (VARLEN && ((smask >> (uint32_t)(t - ts)) & 1u)) {
#pragma unroll
            for (int n = 0; n < NS; ++n) h[n] = 0.f;
          }
          float Bv[NS];
          BCLoad<Tbc>::template row<NS>(Bbase + t * Bstep, Bv);
          const float uu = Elem<Tio>::load(p.u, ub + t * p.su[2]);
          float dt = Elem<Tio>::load(p.delta, db + t * p.sdl[2]) + bias;
          if (p.softplus) dt = softplus20(dt);
          const float dtu = dt * uu;
#pragma unroll
          for (int n = 0; n < NS; ++n) h[n] = fmaf(fast_exp2(dt * Ap[n]), h[n], dtu * Bv[n]);
        }
      }
    }
    // Reverse over segments.
    for (int k = NSEG - 1; k >= 0; --k) {
      const int64_t sg0 = ts + k * SEG;
      if (sg0 >= te) continue;
      float hs[SEG][NS];
      float uus[SEG], dts[SEG], pres[SEG];
#pragma unroll
      for (int n = 0; n < NS; ++n) h[n] = s_seg[k][n][tid];
#pragma unroll
      for (int i = 0; i < SEG; ++i) {
        const int64_t t = sg0 + i;
        if (t < te) {
          if (VARLEN && ((smask >> (uint32_t)(t - ts)) & 1u)) {
#pragma unroll
            for (int n = 0; n < NS; ++n) h[n] = 0.f;
          }
          float Bv[NS];
          BCLoad<Tbc>::template row<NS>(Bbase + t * Bstep, Bv);
          const float uu = Elem<Tio>::load(p.u, ub + t * p.su[2]);
          const float pre = Elem<Tio>::load(p.delta, db + t * p.sdl[2]) + bias;
          const float dt = p.softplus ? softplus20(pre) : pre;
          const float dtu = dt * uu;
#pragma unroll
          for (int n = 0; n < NS; ++n) {
            h[n] = fmaf(fast_exp2(dt * Ap[n]), h[n], dtu * Bv[n]);
            hs[i][n] = h[n];
          }
          uus[i] = uu;
          dts[i] = dt;
          pres[i] = pre;
        }
      }
#pragma unroll
      for (int i = SEG - 1; i >= 0; --i) {
        const int64_t t = sg0 + i;
        if (t < te) {
          const bool st = VARLEN ? (((smask >> (uint32_t)(t - ts)) & 1u) != 0) : (t == 0);
          float Bv[NS], Cv[NS];
          BCLoad<Tbc>::template row<NS>(Bbase + t * Bstep, Bv);
          BCLoad<Tbc>::template row<NS>(Cbase + t * Cstep, Cv);
          const float uu = uus[i], dt = dts[i];
          const float dtu = dt * uu;
          const float dov = Elem<Tio>::load(p.dout, dob + t * p.sdo[2]);
          float dy = dov;
          if (p.has_z) {
            const float zz = Elem<Tio>::load(p.z, zb + t * p.sz[2]);
            const float sg = sigmoidf_(zz);
            dy = dov * (zz * sg);
            const float yo = Elem<Tio>::load(p.out, oub + t * p.sout[2]);
            if (active) Elem<Tio>::store(p.dz, dzb + t * p.sdz[2], dov * yo * sg * (1.f + zz * (1.f - sg)));
          }
          float hp[NS];
          if (i > 0) {
#pragma unroll
            for (int n = 0; n < NS; ++n) hp[n] = hs[i - 1][n];
          } else {
#pragma unroll
            for (int n = 0; n < NS; ++n) hp[n] = s_seg[k][n][tid];
          }
          float s1 = 0.f, s2 = 0.f;
          float pB[NS], pC[NS];
#pragma unroll
          for (int n = 0; n < NS; ++n) {
            const float a = fast_exp2(dt * Ap[n]);
            const float lam = fmaf(Cv[n], dy, gs[n]);
            const float q = st ? 0.f : lam * (a * hp[n]);
            dAacc[n] = fmaf(q, dt, dAacc[n]);
            s2 = fmaf(q, Ap[n], s2);
            s1 = fmaf(lam, Bv[n], s1);
            pB[n] = active ? lam * dtu : 0.f;
            pC[n] = active ? dy * hs[i][n] : 0.f;
            gs[n] = st ? 0.f : a * lam;
          }
          s2 *= 0.69314718055994531f;  // Ap = A * log2(e)
          const float duv = fmaf(dt, s1, Dv * dy);
          float ddv = fmaf(uu, s1, s2);
          if (p.softplus) ddv *= softplus20_grad(pres[i]);
          if (active) {
            Elem<Tio>::store(p.du, dub + t * p.sdu[2], duv);
            Elem<Tio>::store(p.ddelta, ddb + t * p.sddl[2], ddv);
          }
          dDacc = fmaf(dy, uu, dDacc);
          dbacc += ddv;
          wave_transpose_reduce16(pB, lane);
          wave_transpose_reduce16(pC, lane);
          if ((lane & 3) == 0) {
            s_red[0][i][wv][lane >> 2] = pB[0];
            s_red[1][i][wv][lane >> 2] = pC[0];
          }
        }
      }
      __syncthreads();
      {
        const int which = tid >> 7;
        const int i = (tid >> 4) & 7;
        const int n = tid & 15;
        const int64_t t = sg0 + i;
        if (t < te && n < N) {
          const float v = s_red[which][i][0][n] + s_red[which][i][1][n] + s_red[which][i][2][n] +
                          s_red[which][i][3][n];
          (which ? pCrow : pBrow)[t * p.N + n] = v;
        }
      }
      __syncthreads();
    }
  }
  if (active) {
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) atomicAdd(p.dA + d * p.sdA[0] + n * p.sdA[1], dAacc[n]);
    if (p.has_D) atomicAdd(p.dD + d * p.sdD, dDacc);
    if (p.has_bias) atomicAdd(p.dbias + d * p.sdbias, dbacc);
  }
}

// dB[b, g, n, t] = sum over 256-channel blocks of the partials.
__global__ void __launch_bounds__(256) bwd_reduce_bc(BwdK p) {
  const int64_t total = p.Bsz * p.G * p.L * p.N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i % p.N;
    int64_t r = i / p.N;
    const int64_t t = r % p.L;
    r /= p.L;
    const int64_t g = r % p.G;
    const int64_t b = r / p.G;
    const int64_t base = (b * p.G + g) * p.nJ4;
    float sb = 0.f, sc = 0.f;
    for (int64_t j = 0; j < p.nJ4; ++j) {
      sb += p.ws_pB[((base + j) * p.L + t) * p.N + n];
      sc += p.ws_pC[((base + j) * p.L + t) * p.N + n];
    }
    p.dB[b * p.sdB[0] + g * p.sdB[1] + n * p.sdB[2] + t * p.sdB[3]] = sb;
    p.dC[b * p.sdC[0] + g * p.sdC[1] + n * p.sdC[2] + t * p.sdC[3]] = sc;
  }
}

static hipError_t record(void* const* ev, int i, hipStream_t st) {
  if (ev == nullptr || ev[i] == nullptr) return hipSuccess;
  return hipEventRecord((hipEvent_t)ev[i], st);
}

template <typename Tio, typename Tbc, bool VARLEN>
static hipError_t launch_bwd_t(const BwdK& k, hipStream_t st, void* const* ev) {
  hipError_t e;
  if (k.K > 1) {
    dim3 grid((unsigned)(k.Bsz * k.nDblk), (unsigned)(k.K - 1));
    hipLaunchKernelGGL((bwd_summary<Tio, Tbc, 16, VARLEN>), grid, dim3(kWave), 0, st, k);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int64_t total = k.Bsz * k.D * k.N;
    hipLaunchKernelGGL(bwd_carry, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, k);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  dim3 grid((unsigned)(k.Bsz * k.G * k.nJ4), (unsigned)k.K);
  if ((e = record(ev, 0, st)) != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_main<Tio, Tbc, VARLEN>), grid, dim3(256), 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = record(ev, 1, st)) != hipSuccess) return e;
  const int64_t total = k.Bsz * k.G * k.L * k.N;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(bwd_reduce_bc, dim3((unsigned)blocks), dim3(256), 0, st, k);
  return hipGetLastError();
}

template <typename Tio, typename Tbc>
static hipError_t launch_bwd_v(const BwdK& k, hipStream_t st, void* const* ev) {
  return k.nseq > 0 ? launch_bwd_t<Tio, Tbc, true>(k, st, ev)
                    : launch_bwd_t<Tio, Tbc, false>(k, st, ev);
}

template <typename Tio>
static hipError_t launch_bwd_io(const BwdK& k, int bc_dtype, hipStream_t st, void* const* ev) {
  switch (bc_dtype) {
    case S6_F32: return launch_bwd_v<Tio, float>(k, st, ev);
    case S6_BF16: return launch_bwd_v<Tio, bf16>(k, st, ev);
    default: return launch_bwd_v<Tio, f16>(k, st, ev);
  }
}

hipError_t launch_bwd(const BwdK& k, int io_dtype, int bc_dtype, hipStream_t st, void* const* ev) {
  switch (io_dtype) {
    case S6_F32: return launch_bwd_io<float>(k, bc_dtype, st, ev);
    case S6_BF16: return launch_bwd_io<bf16>(k, bc_dtype, st, ev);
    default: return launch_bwd_io<f16>(k, bc_dtype, st, ev);
  }
}

}  // namespace s6
