// Forward S6 selective scan for gfx950.
//
// Mapping: one lane owns one channel (b, d) and keeps all of its N states in VGPRs; a
// 64-lane workgroup covers 64 channels of one (batch, group).  B_t and C_t are identical
// for every lane of the workgroup, so they are read through the scalar cache into SGPRs
// and feed v_fma directly.  The sequence is cut into K chunks of Lc steps so that
// B * D / 64 * K waves fill the chip:
//   fwd_scan<FULL=false>  chunk summary: state of each chunk from a zero start and the sum
//                         of Delta since its last sequence start          (chunks 0..K-2)
//   fwd_carry             prefix over chunks: h_in(c+1) = exp(A * S_c) h_in(c) + h_loc(c)
//   fwd_scan<FULL=true>   rescan each chunk from its carried-in state, fused with
//                         y = C h + D u, the silu(z) gate, checkpoints and last states.
// The recurrence and its rounding points follow selective_scan_ref
// (selective_scan_interface.py:107-156): Delta = softplus(delta + bias) in fp32,
// abar = exp(Delta * A), h = abar * h + Delta * u * B, y = sum_n C h + D u.
#include "s6_internal.h"

namespace s6 {

// Sequence bookkeeping for packed varlen input.  `pending` is the first sequence start
// >= t (or > L when none is left) and `seq` the index of the sequence that owns step t.
struct SeqCursor {
  int32_t idx;      // index into cu_seqlens of `pending`
  int64_t pending;
};

__device__ inline SeqCursor seq_cursor_at(const int32_t* cu, int32_t nseq, int64_t t0) {
  // first i with cu[i] >= t0  (cu is non-decreasing, cu[0] = 0, cu[nseq] = L)
  int32_t lo = 0, hi = nseq + 1;
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if ((int64_t)cu[mid] < t0) lo = mid + 1; else hi = mid;
  }
  SeqCursor s;
  s.idx = lo;
  s.pending = (lo <= nseq) ? (int64_t)cu[lo] : INT64_MAX;
  return s;
}

template <typename Tio, typename Tbc, int NS, bool FULL, bool VARLEN>
__global__ void __launch_bounds__(kWave) fwd_scan(FwdK p) {
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
  const int64_t c = blockIdx.y;
  const int64_t t0 = c * p.Lc;
  const int64_t t1 = min(t0 + p.Lc, p.L);
  const int N = (int)p.N;
  constexpr int ES = Elem<Tio>::kSize;

  float Ap[NS];
  float h[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    Ap[n] = (n < N) ? p.A[d * p.sA[0] + n * p.sA[1]] * kLog2e : 0.f;
    h[n] = 0.f;
  }
  const int64_t ch = b * p.D + d;  // channel index for workspaces / checkpoints
  if (FULL && c > 0) {
    const float* hin = p.ws_h + (ch * p.K + c) * p.N;
#pragma unroll
    for (int n = 0; n < NS; ++n) h[n] = (n < N) ? hin[n] : 0.f;
  }
  const float bias = p.has_bias ? p.bias[d * p.sbias] : 0.f;
  const float Dv = (FULL && p.has_D) ? p.Dp[d * p.sD] : 0.f;

  // Per-lane byte pointers, advanced by one time step per iteration.
  const char* up = (const char*)p.u + (b * p.su[0] + d * p.su[1] + t0 * p.su[2]) * ES;
  const char* dp = (const char*)p.delta + (b * p.sdl[0] + d * p.sdl[1] + t0 * p.sdl[2]) * ES;
  const char* zp = FULL && p.has_z ? (const char*)p.z + (b * p.sz[0] + d * p.sz[1] + t0 * p.sz[2]) * ES : nullptr;
  char* op = FULL ? (char*)p.out + (b * p.so[0] + d * p.so[1] + t0 * p.so[2]) * ES : nullptr;
  char* ozp = FULL && p.has_z ? (char*)p.out_z + (b * p.soz[0] + d * p.soz[1] + t0 * p.soz[2]) * ES : nullptr;
  const int64_t ust = p.su[2] * ES, dst = p.sdl[2] * ES, zst = p.sz[2] * ES, ost = p.so[2] * ES,
                ozst = p.soz[2] * ES;
  const char* Brow = (const char*)p.Bm + (b * p.sB[0] + g * p.sB[1] + t0 * p.sB[3]) * Elem<Tbc>::kSize;
  const char* Crow = (const char*)p.Cm + (b * p.sC[0] + g * p.sC[1] + t0 * p.sC[3]) * Elem<Tbc>::kSize;
  const int64_t Bstep = p.sB[3] * Elem<Tbc>::kSize;
  const int64_t Cstep = p.sC[3] * Elem<Tbc>::kSize;
  const bool has_z = FULL && p.has_z;
  const bool softplus = p.softplus != 0;

  SeqCursor sc;
  if (VARLEN) sc = seq_cursor_at(p.cu, p.nseq, t0);
  float ssum = 0.f;  // sum of Delta since the last sequence start (chunk summary only)

  // Blocks of kCk steps end exactly on checkpoint boundaries (t0 is a multiple of kCk).
  for (int64_t tb = t0; tb < t1; tb += kCk) {
    const int64_t te = min(tb + (int64_t)kCk, t1);
    for (int64_t t = tb; t < te; ++t) {
      if (VARLEN && t == sc.pending) {
#pragma unroll
        for (int n = 0; n < NS; ++n) h[n] = 0.f;
        ssum = 0.f;
        while (sc.idx <= p.nseq && (int64_t)p.cu[sc.idx] <= t) ++sc.idx;
        sc.pending = (sc.idx <= p.nseq) ? (int64_t)p.cu[sc.idx] : INT64_MAX;
      }
      float Bv[NS];
      BCLoad<Tbc>::template row<NS>(Brow, Bv);
      Brow += Bstep;
      float Cv[NS];
      if (FULL) {
        BCLoad<Tbc>::template row<NS>(Crow, Cv);
        Crow += Cstep;
      }
      const float uu = Elem<Tio>::load(up, 0);
      float dt = Elem<Tio>::load(dp, 0) + bias;
      up += ust;
      dp += dst;
      if (softplus) dt = softplus20(dt);
      const float dtu = dt * uu;
      float y = 0.f;
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        const float a = fast_exp2(dt * Ap[n]);
        h[n] = fmaf(a, h[n], dtu * Bv[n]);
        if (FULL) y = fmaf(Cv[n], h[n], y);
      }
      if (!FULL) {
        ssum += dt;
      } else {
        y = fmaf(uu, Dv, y);
        if (active) Elem<Tio>::store(op, 0, y);
        op += ost;
        if (has_z) {
          const float zz = Elem<Tio>::load(zp, 0);
          if (active) Elem<Tio>::store(ozp, 0, y * zz * sigmoidf_(zz));
          zp += zst;
          ozp += ozst;
        }
        if (VARLEN && p.last_state != nullptr && active && (t + 1 == sc.pending || t == p.L - 1)) {
          float* ls = p.last_state + ((int64_t)(sc.idx - 1) * p.D + d) * p.N;
#pragma unroll
          for (int n = 0; n < NS; ++n)
            if (n < N) ls[n] = h[n];
        }
      }
    }
    if (FULL && active) {
      if (p.x_ckpt != nullptr) {
        float* xc = p.x_ckpt + (ch * p.nck + (te - 1) / kCk) * p.N;
#pragma unroll
        for (int n = 0; n < NS; ++n)
          if (n < N) xc[n] = h[n];
      }
      if (!VARLEN && p.last_state != nullptr && te == p.L) {
        float* ls = p.last_state + ch * p.N;
#pragma unroll
        for (int n = 0; n < NS; ++n)
          if (n < N) ls[n] = h[n];
      }
    }
  }
  if (!FULL && active) {
    float* ho = p.ws_h + (ch * p.K + c) * p.N;
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) ho[n] = h[n];
    p.ws_s[ch * p.K + c] = ssum;
  }
}

// Prefix over chunk summaries, one thread per (channel, n).  Replaces each summary with
// the state carried into its chunk.
__global__ void __launch_bounds__(256) fwd_carry(FwdK p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = p.Bsz * p.D * p.N;
  if (i >= total) return;
  const int64_t ch = i / p.N;
  const int64_t n = i % p.N;
  const int64_t d = ch % p.D;
  const float ap = p.A[d * p.sA[0] + n * p.sA[1]] * kLog2e;
  float carry = 0.f;
  for (int64_t c = 0; c < p.K; ++c) {
    float* slot = p.ws_h + (ch * p.K + c) * p.N + n;
    const float hloc = (c + 1 < p.K) ? *slot : 0.f;
    *slot = carry;
    if (c + 1 < p.K) {
      bool reset = false;
      if (p.nseq > 0) {
        const int64_t t0 = c * p.Lc, t1 = min(t0 + p.Lc, p.L);
        SeqCursor s = seq_cursor_at(p.cu, p.nseq, t0);
        reset = s.pending < t1;
      }
      const float decay = fast_exp2(ap * p.ws_s[ch * p.K + c]);
      carry = (reset ? 0.f : decay * carry) + hloc;
    }
  }
}

__global__ void fill_f32(float* __restrict__ p, int64_t n, float v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = v;
}

// Copy B or C ([batch, G, N, L], any strides) into a dense [batch, G, L, NP] buffer of the
// same element type so the scan can read each time step as one scalar-cache row.
template <typename T>
__global__ void relayout_bc(const T* __restrict__ src, int64_t s0, int64_t s1, int64_t s2,
                            int64_t s3, T* __restrict__ dst, int64_t Bsz, int64_t G, int64_t N,
                            int64_t NP, int64_t L) {
  const int64_t total = Bsz * G * L * NP;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i % NP;
    int64_t r = i / NP;
    const int64_t t = r % L; r /= L;
    const int64_t g = r % G;
    const int64_t b = r / G;
    T v{};
    if (n < N) v = src[b * s0 + g * s1 + n * s2 + t * s3];
    dst[i] = v;
  }
}

// ---------------------------------------------------------------------------------------
// Host-side launch helpers
// ---------------------------------------------------------------------------------------

template <typename Tio, typename Tbc, int NS, bool VARLEN>
static hipError_t launch_scan_pair(const FwdK& k, hipStream_t st) {
  if (k.K > 1) {
    dim3 grid((unsigned)(k.Bsz * k.nDblk), (unsigned)(k.K - 1));
    hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, false, VARLEN>), grid, dim3(kWave), 0, st, k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t total = k.Bsz * k.D * k.N;
    hipLaunchKernelGGL(fwd_carry, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, k);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  dim3 grid((unsigned)(k.Bsz * k.nDblk), (unsigned)k.K);
  hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, true, VARLEN>), grid, dim3(kWave), 0, st, k);
  return hipGetLastError();
}

template <typename Tio, typename Tbc, int NS>
static hipError_t launch_ns(const FwdK& k, hipStream_t st) {
  return k.nseq > 0 ? launch_scan_pair<Tio, Tbc, NS, true>(k, st)
                    : launch_scan_pair<Tio, Tbc, NS, false>(k, st);
}

template <typename Tio, typename Tbc>
static hipError_t launch_bc(const FwdK& k, hipStream_t st) {
  if (k.N <= 8) return launch_ns<Tio, Tbc, 8>(k, st);
  if (k.N <= 16) return launch_ns<Tio, Tbc, 16>(k, st);
  if (k.N <= 32) return launch_ns<Tio, Tbc, 32>(k, st);
  return launch_ns<Tio, Tbc, 64>(k, st);
}

template <typename Tio>
static hipError_t launch_io(const FwdK& k, int bc_dtype, hipStream_t st) {
  switch (bc_dtype) {
    case S6_F32: return launch_bc<Tio, float>(k, st);
    case S6_BF16: return launch_bc<Tio, bf16>(k, st);
    default: return launch_bc<Tio, f16>(k, st);
  }
}

hipError_t launch_fwd(const FwdK& k, int io_dtype, int bc_dtype, hipStream_t st) {
  switch (io_dtype) {
    case S6_F32: return launch_io<float>(k, bc_dtype, st);
    case S6_BF16: return launch_io<bf16>(k, bc_dtype, st);
    default: return launch_io<f16>(k, bc_dtype, st);
  }
}

hipError_t launch_fill(float* p, int64_t n, float v, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(fill_f32, dim3((unsigned)blocks), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

hipError_t launch_relayout(const void* src, const int64_t s[4], int esize, void* dst,
                           int64_t Bsz, int64_t G, int64_t N, int64_t NP, int64_t L,
                           hipStream_t st) {
  const int64_t total = Bsz * G * L * NP;
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  if (esize == 4)
    hipLaunchKernelGGL(relayout_bc<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint32_t*)src, s[0], s[1], s[2], s[3], (uint32_t*)dst, Bsz, G, N,
                       NP, L);
  else
    hipLaunchKernelGGL(relayout_bc<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint16_t*)src, s[0], s[1], s[2], s[3], (uint16_t*)dst, Bsz, G, N,
                       NP, L);
  return hipGetLastError();
}

}  // namespace s6
