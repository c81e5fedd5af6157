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

// Stores n < N states of one lane (NS registers) to a contiguous fp32 row.
template <int NS>
__device__ inline void store_state(float* dst, const float (&h)[NS], int N) {
  if (N == NS && (NS % 4) == 0) {
#pragma unroll
    for (int n = 0; n < NS; n += 4)
      *reinterpret_cast<float4*>(dst + n) = make_float4(h[n], h[n + 1], h[n + 2], h[n + 3]);
  } else {
    for (int n = 0; n < N; ++n) dst[n] = h[n];  // N < NS: dynamic count, rare
  }
}

// MODE 0: chunk summary; 1: output pass; 2: output pass with the silu(z) gate.
template <typename Tio, typename Tbc, int NS, int MODE, bool VARLEN>
__global__ void __launch_bounds__(kWave) fwd_scan(FwdK p) {
  constexpr bool FULL = MODE != 0;
  constexpr bool HAS_Z = MODE == 2;
  constexpr int TB = 8;  // time steps per unrolled block; divides kCk
  constexpr int ES = Elem<Tio>::kSize;
  constexpr int G = NS < 32 / Elem<Tbc>::kSize ? NS : 32 / Elem<Tbc>::kSize;  // 8 words per scalar-cache group
  constexpr int NG = NS / G;
  constexpr int EB = Elem<Tbc>::kSize;
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
  const int64_t d0 = g * Dg + j * kWave;  // first channel of this wave
  const int64_t d = g * Dg + (active ? dloc : Dg - 1);
  const int c = blockIdx.y;
  const int L = (int)p.L;
  const int t0 = c * (int)p.Lc;
  const int t1 = min(t0 + (int)p.Lc, L);
  const int N = (int)p.N;

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
  const bool has_bias = p.has_bias != 0;
  const float bias = has_bias ? p.bias[d * p.sbias] : 0.f;
  const float Dv = (FULL && p.has_D) ? p.Dp[d * p.sD] : 0.f;
  constexpr bool has_z = HAS_Z;
  const bool softplus = p.softplus != 0;
  float* const xck = (FULL && p.x_ckpt != nullptr && active) ? p.x_ckpt + ch * p.nck * p.N : nullptr;

  // Buffer resources based at (b, d0, t0) of each [batch, dim, seqlen] tensor.
  const auto rs_u = make_rsrc((const char*)p.u + (b * p.su[0] + d0 * p.su[1] + (int64_t)t0 * p.su[2]) * ES);
  const auto rs_d = make_rsrc((const char*)p.delta + (b * p.sdl[0] + d0 * p.sdl[1] + (int64_t)t0 * p.sdl[2]) * ES);
  const uint32_t vo_u = active ? (uint32_t)(lane * p.su[1] * ES) : kOffDrop;
  const uint32_t vo_d = active ? (uint32_t)(lane * p.sdl[1] * ES) : kOffDrop;
  const uint32_t st_u = (uint32_t)(p.su[2] * ES), st_d = (uint32_t)(p.sdl[2] * ES);
  // Unused resources (no output in the summary pass, no z) point at u and are never read.
  const auto rs_o = make_rsrc(FULL ? (const char*)p.out + (b * p.so[0] + d0 * p.so[1] + (int64_t)t0 * p.so[2]) * ES
                                   : (const char*)p.u);
  const auto rs_z = make_rsrc(has_z ? (const char*)p.z + (b * p.sz[0] + d0 * p.sz[1] + (int64_t)t0 * p.sz[2]) * ES
                                    : (const char*)p.u);
  const auto rs_oz = make_rsrc(has_z ? (const char*)p.out_z + (b * p.soz[0] + d0 * p.soz[1] + (int64_t)t0 * p.soz[2]) * ES
                                     : (const char*)p.u);
  const uint32_t vo_o = (FULL && active) ? (uint32_t)(lane * p.so[1] * ES) : kOffDrop;
  const uint32_t vo_z = (has_z && active) ? (uint32_t)(lane * p.sz[1] * ES) : kOffDrop;
  const uint32_t vo_oz = (has_z && active) ? (uint32_t)(lane * p.soz[1] * ES) : kOffDrop;
  const uint32_t st_o = FULL ? (uint32_t)(p.so[2] * ES) : 0u;
  const uint32_t st_z = has_z ? (uint32_t)(p.sz[2] * ES) : 0u;
  const uint32_t st_oz = has_z ? (uint32_t)(p.soz[2] * ES) : 0u;
  // B / C rows of this wave's (batch, group), from step t0; 32-bit byte offsets per step.
  const char* const Bbase = (const char*)p.Bm + (b * p.sB[0] + g * p.sB[1] + (int64_t)t0 * p.sB[3]) * EB;
  const char* const Cbase = (const char*)p.Cm + (b * p.sC[0] + g * p.sC[1] + (int64_t)t0 * p.sC[3]) * EB;
  const uint32_t Bst = (uint32_t)(p.sB[3] * EB), Cst = (uint32_t)(p.sC[3] * EB);

  SeqCursor sc;
  if (VARLEN) sc = seq_cursor_at(p.cu, p.nseq, t0);
  float ssum = 0.f;  // sum of Delta since the last sequence start (chunk summary only)

  // Register double buffer: the next block's u / delta / z are in flight while the
  // current block computes.  Loads past t1 re-read step t1 - 1.
  float un[TB], dn[TB], zn[TB];
  auto fetch = [&](int tb) {
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      const uint32_t r = (uint32_t)(min(tb + i, t1 - 1) - t0);
      un[i] = Buf<Tio>::load(rs_u, vo_u, r * st_u);
      dn[i] = Buf<Tio>::load(rs_d, vo_d, r * st_d);
      if (has_z) zn[i] = Buf<Tio>::load(rs_z, vo_z, r * st_z);
    }
  };
  fetch(t0);

  // B_t / C_t arrive through the scalar cache one group of G states ahead of their use;
  // the scheduling barrier after each group keeps the compiler from hoisting every row of
  // the unrolled block into SGPRs at once.
  BCGroup<Tbc> bnx, cnx;
  bnx.template load<G>(Bbase);
  if (FULL) cnx.template load<G>(Cbase);

  for (int tb = t0; tb < t1; tb += TB) {
    float uc[TB], dc[TB], zc[TB];
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      uc[i] = un[i];
      dc[i] = dn[i];
      zc[i] = has_z ? zn[i] : 0.f;
    }
    if (tb + TB < t1) fetch(tb + TB);
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      const int t = tb + i;
      if (t < t1) {
        if (VARLEN && t == sc.pending) {
#pragma unroll
          for (int n = 0; n < NS; ++n) h[n] = 0.f;
          ssum = 0.f;
          while (sc.idx <= p.nseq && (int64_t)p.cu[sc.idx] <= t) ++sc.idx;
          sc.pending = (sc.idx <= p.nseq) ? (int64_t)p.cu[sc.idx] : INT64_MAX;
        }
        const uint32_t r = (uint32_t)(t - t0);
        const uint32_t rn = (uint32_t)(min(t + 1, t1 - 1) - t0);
        const float uu = uc[i];
        float dt = dc[i];
        if (has_bias) dt += bias;
        if (softplus) dt = softplus20(dt);
        const float dtu = dt * uu;
        // y accumulates in 4 independent FMA chains (n mod 4): shorter dependency chains
        // and a smaller rounding error than one long chain.
        float ys[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          const BCGroup<Tbc> bcur = bnx;
          BCGroup<Tbc> ccur;
          if (FULL) ccur = cnx;
          if (gi + 1 < NG) {
            bnx.template load<G>(Bbase + r * Bst + (gi + 1) * G * EB);
            if (FULL) cnx.template load<G>(Cbase + r * Cst + (gi + 1) * G * EB);
          } else {
            bnx.template load<G>(Bbase + rn * Bst);
            if (FULL) cnx.template load<G>(Cbase + rn * Cst);
          }
#pragma unroll
          for (int k = 0; k < G; ++k) {
            const int n = gi * G + k;
            const float a = fast_exp2(dt * Ap[n]);
            h[n] = fmaf(a, h[n], dtu * bcur.get(k));
            if (FULL) ys[k & 3] = (gi == 0 && k < 4) ? ccur.get(k) * h[n] : fmaf(ccur.get(k), h[n], ys[k & 3]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (!FULL) {
          ssum += dt;
        } else {
          float y = (ys[0] + ys[1]) + (ys[2] + ys[3]);
          y = fmaf(uu, Dv, y);
          Buf<Tio>::store(rs_o, vo_o, r * st_o, y);
          if (has_z) {
            const float zz = zc[i];
            Buf<Tio>::store(rs_oz, vo_oz, r * st_oz, y * zz * sigmoidf_(zz));
          }
          if (VARLEN && p.last_state != nullptr && active && (t + 1 == sc.pending || t == L - 1))
            store_state<NS>(p.last_state + ((int64_t)(sc.idx - 1) * p.D + d) * p.N, h, N);
          if (((t + 1) & (kCk - 1)) == 0 || t == L - 1) {
            if (xck != nullptr) store_state<NS>(xck + (int64_t)(t / kCk) * p.N, h, N);
            if (!VARLEN && p.last_state != nullptr && active && t == L - 1)
              store_state<NS>(p.last_state + ch * p.N, h, N);
          }
        }
      }
    }
  }
  if (!FULL && active) {
    store_state<NS>(p.ws_h + (ch * p.K + c) * p.N, h, N);
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

static hipError_t record(void* const* ev, int i, hipStream_t st) {
  if (ev == nullptr || ev[i] == nullptr) return hipSuccess;
  return hipEventRecord((hipEvent_t)ev[i], st);
}

template <typename Tio, typename Tbc, int NS, bool VARLEN>
static hipError_t launch_scan_pair(const FwdK& k, hipStream_t st, void* const* ev) {
  hipError_t e = hipSuccess;
  if (k.K > 1) {
    dim3 grid((unsigned)(k.Bsz * k.nDblk), (unsigned)(k.K - 1));
    hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, 0, VARLEN>), grid, dim3(kWave), 0, st, k);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t total = k.Bsz * k.D * k.N;
    hipLaunchKernelGGL(fwd_carry, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, k);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  dim3 grid((unsigned)(k.Bsz * k.nDblk), (unsigned)k.K);
  e = record(ev, 0, st);
  if (e != hipSuccess) return e;
  if (k.has_z)
    hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, 2, VARLEN>), grid, dim3(kWave), 0, st, k);
  else
    hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, 1, VARLEN>), grid, dim3(kWave), 0, st, k);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return record(ev, 1, st);
}

template <typename Tio, typename Tbc, int NS>
static hipError_t launch_ns(const FwdK& k, hipStream_t st, void* const* ev) {
  return k.nseq > 0 ? launch_scan_pair<Tio, Tbc, NS, true>(k, st, ev)
                    : launch_scan_pair<Tio, Tbc, NS, false>(k, st, ev);
}

template <typename Tio, typename Tbc>
static hipError_t launch_bc(const FwdK& k, hipStream_t st, void* const* ev) {
  if (k.N <= 8) return launch_ns<Tio, Tbc, 8>(k, st, ev);
  if (k.N <= 16) return launch_ns<Tio, Tbc, 16>(k, st, ev);
  if (k.N <= 32) return launch_ns<Tio, Tbc, 32>(k, st, ev);
  return launch_ns<Tio, Tbc, 64>(k, st, ev);
}

template <typename Tio>
static hipError_t launch_io(const FwdK& k, int bc_dtype, hipStream_t st, void* const* ev) {
  switch (bc_dtype) {
    case S6_F32: return launch_bc<Tio, float>(k, st, ev);
    case S6_BF16: return launch_bc<Tio, bf16>(k, st, ev);
    default: return launch_bc<Tio, f16>(k, st, ev);
  }
}

hipError_t launch_fwd(const FwdK& k, int io_dtype, int bc_dtype, hipStream_t st, void* const* ev) {
  switch (io_dtype) {
    case S6_F32: return launch_io<float>(k, bc_dtype, st, ev);
    case S6_BF16: return launch_io<bf16>(k, bc_dtype, st, ev);
    default: return launch_io<f16>(k, bc_dtype, st, ev);
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
