// Small kernels around the S6 scans: the inter-chunk carries of the forward and backward
// passes, the deterministic reductions of the backward's partial sums, fills, the B/C
// relayout, and the dispatch over the input dtype.
#include "s6_internal.h"

namespace s6 {

// Inter-chunk carry, in place.  Chunk c contributes the affine map  x -> m_c x + loc_c
// (m_c = 0 when a sequence starts inside chunk c, else exp(A S_c) with S_c the chunk's sum
// of Delta); the maps are composed in chunk order (forward: c = 0, 1, ...; REV:
// c = K-1, K-2, ...).  One thread per (channel, state); the chunk values are loaded 16 at a
// time before the sequential composition, so a thread waits for one load round trip per
// 16 chunks.
//   forward: ws[ch, c] = state chunk c reaches from a zero start -> state carried into c
//   REV:     ws[ch, c] = gradient chunk c passes out of its first step from a zero inflow
//            -> gradient flowing into chunk c from chunk c + 1
// The chunk composed last (forward: c = K-1; REV: c = 0) has no summary of its own.
// The group's loads are unconditional, from chunk min(step, K - 2) (in bounds), and the steps
// past K - 2 are masked at use: a load under a branch (as `has ? ws[..] : 0` compiles to)
// waits for itself before the branch joins, one round trip per chunk.
template <bool REV, bool VARLEN>
__global__ void __launch_bounds__(256) chunk_carry(CarryK p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.nch * p.N) return;
  const int64_t ch = i / p.N, n = i % p.N;
  const int64_t d = ch % p.D;
  const int64_t K = p.K;
  if (K < 2) {  // one chunk: nothing flows into it
    p.ws[ch * K * p.N + n] = 0.f;
    return;
  }
  const float ap = p.A[d * p.sA[0] + n * p.sA[1]] * kLog2e;
  constexpr int G = 16;
  float carry = 0.f;
  for (int64_t s0 = 0; s0 < K; s0 += G) {
    float hl[G], S[G];
    int rs[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int64_t step = min(s0 + k, K - 2);
      const int64_t c = REV ? K - 1 - step : step;
      hl[k] = p.ws[(ch * K + c) * p.N + n];
      S[k] = p.ws_s[ch * K + c];
      rs[k] = VARLEN ? p.ws_r[ch * K + c] : 0;
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int64_t step = s0 + k;
      if (step < K) {
        const int64_t c = REV ? K - 1 - step : step;
        p.ws[(ch * K + c) * p.N + n] = carry;  // value entering chunk c
        if (step < K - 1) carry = rs[k] ? hl[k] : fmaf(fast_exp2(ap * S[k]), carry, hl[k]);
      }
    }
  }
}

// dB[b, g, n, t] (dC likewise) = sum over the 64-channel blocks j of the partials
// ws_pB[b, g, j, t, 0:NPr]; one thread per (b, g, t), fixed summation order.
__global__ void __launch_bounds__(256) bwd_reduce_bc(BwdK p) {
  constexpr int W = kBwdGroup;
  const int64_t total = p.Bsz * p.G * p.L;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i % p.L;
    const int64_t bg = i / p.L;
    const int64_t b = bg / p.G, g = bg % p.G;
    for (int64_t n0 = 0; n0 < p.NPr; n0 += W) {
      float sb[W], sc[W];
#pragma unroll
      for (int n = 0; n < W; ++n) sb[n] = sc[n] = 0.f;
      // Rows in groups of RG: the group's loads are issued together (in flight at once), then
      // added in row order j = 0, 1, ... (the result does not depend on the grouping).
      constexpr int RG = 4;
      for (int64_t j0 = 0; j0 < p.nJ; j0 += RG) {
        float4 vb[RG][W / 4], vc[RG][W / 4];
#pragma unroll
        for (int r = 0; r < RG; ++r) {
          const int64_t j = min(j0 + r, p.nJ - 1);  // in bounds; rows past nJ are not added
          const int64_t row = ((bg * p.nJ + j) * p.L + t) * p.NPr + n0;
#pragma unroll
          for (int q = 0; q < W / 4; ++q) {
            vb[r][q] = *reinterpret_cast<const float4*>(p.ws_pB + row + 4 * q);
            vc[r][q] = *reinterpret_cast<const float4*>(p.ws_pC + row + 4 * q);
          }
        }
#pragma unroll
        for (int r = 0; r < RG; ++r) {
          // rows past nJ add an exact 0 (a select, not a branch, which would let the compiler
          // sink the group's loads behind each other)
          const bool on = j0 + r < p.nJ;
#pragma unroll
          for (int q = 0; q < W / 4; ++q) {
            const int n = 4 * q;
            const float4 b4 = vb[r][q], c4 = vc[r][q];
            sb[n] += on ? b4.x : 0.f; sb[n + 1] += on ? b4.y : 0.f;
            sb[n + 2] += on ? b4.z : 0.f; sb[n + 3] += on ? b4.w : 0.f;
            sc[n] += on ? c4.x : 0.f; sc[n + 1] += on ? c4.y : 0.f;
            sc[n + 2] += on ? c4.z : 0.f; sc[n + 3] += on ? c4.w : 0.f;
          }
        }
      }
#pragma unroll
      for (int n = 0; n < W; ++n) {
        const int64_t nn = n0 + n;
        if (nn < p.N) {
          p.dB[b * p.sdB[0] + g * p.sdB[1] + nn * p.sdB[2] + t * p.sdB[3]] = sb[n];
          p.dC[b * p.sdC[0] + g * p.sdC[1] + nn * p.sdC[2] + t * p.sdC[3]] = sc[n];
        }
      }
    }
  }
}

// dA[d, n], dD[d], ddelta_bias[d]: sums over the Bsz*K (batch, chunk) partial rows.  A block
// of 64 columns x 16 row slices; each slice sums its rows in order, then the 16 slice sums
// are added in slice order (fixed order: deterministic).  blockIdx.y selects dA / dD / dbias.
__global__ void __launch_bounds__(1024) bwd_reduce_params(BwdK p) {
  __shared__ float part[16][64];
  const int col_l = threadIdx.x & 63;
  const int slice = threadIdx.x >> 6;
  const int which = blockIdx.y;
  const int64_t ncol = which == 0 ? p.D * p.N : p.D;
  const float* src = which == 0 ? p.ws_dA : (which == 1 ? p.ws_dD : p.ws_db);
  if (which == 1 && !p.has_D) return;
  if (which == 2 && !p.has_bias) return;
  const int64_t col = (int64_t)blockIdx.x * 64 + col_l;
  if ((int64_t)blockIdx.x * 64 >= ncol) return;
  const int64_t rows = p.Bsz * p.K;
  float s = 0.f;
  if (col < ncol)
    for (int64_t r = slice; r < rows; r += 16) s += src[r * ncol + col];
  part[slice][col_l] = s;
  __syncthreads();
  if (slice == 0 && col < ncol) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += part[k][col_l];
    if (which == 0)
      p.dA[(col / p.N) * p.sdA[0] + (col % p.N) * p.sdA[1]] = t;
    else if (which == 1)
      p.dD[col * p.sdD] = t;
    else
      p.dbias[col * p.sdbias] = t;
  }
}

__global__ void fill_f32(float* __restrict__ p, int64_t n, float v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = v;
}

// Copy B or C ([batch, G, N, L], any strides) into a dense [batch, G, L, NP] buffer of the
// same element type so the scans can read each time step as one scalar-cache row.
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

struct Dims4 {
  int64_t v[4];
};

// dst[i] = src[i] inside sd, 0 outside, for every 4-D index i inside dd; innermost axis fastest.
template <typename T>
__global__ void copy4d(const T* __restrict__ src, Dims4 ss, Dims4 sd, T* __restrict__ dst, Dims4 ds,
                       Dims4 dd) {
  const int64_t total = dd.v[0] * dd.v[1] * dd.v[2] * dd.v[3];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i;
    const int64_t i3 = r % dd.v[3]; r /= dd.v[3];
    const int64_t i2 = r % dd.v[2]; r /= dd.v[2];
    const int64_t i1 = r % dd.v[1];
    const int64_t i0 = r / dd.v[1];
    T v{};
    if (i0 < sd.v[0] && i1 < sd.v[1] && i2 < sd.v[2] && i3 < sd.v[3])
      v = src[i0 * ss.v[0] + i1 * ss.v[1] + i2 * ss.v[2] + i3 * ss.v[3]];
    dst[i0 * ds.v[0] + i1 * ds.v[1] + i2 * ds.v[2] + i3 * ds.v[3]] = v;
  }
}

// ---------------------------------------------------------------------------------------

static unsigned grid_for(int64_t total, int64_t threads) {
  int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 65535) blocks = 65535;
  return (unsigned)(blocks < 1 ? 1 : blocks);
}

template <bool REV>
static hipError_t launch_carry(const CarryK& c, hipStream_t st) {
  const int64_t total = c.nch * c.N;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (c.ws_r != nullptr)
    hipLaunchKernelGGL((chunk_carry<REV, true>), grid, dim3(256), 0, st, c);
  else
    hipLaunchKernelGGL((chunk_carry<REV, false>), grid, dim3(256), 0, st, c);
  return hipGetLastError();
}

hipError_t launch_fwd_carry(const FwdK& k, hipStream_t st) {
  const CarryK c{k.A, {k.sA[0], k.sA[1]}, k.ws_h, k.ws_s, k.ws_r, k.Bsz * k.D, k.D, k.K, k.N};
  return launch_carry<false>(c, st);
}

hipError_t launch_bwd_carry(const BwdK& k, hipStream_t st) {
  const CarryK c{k.A, {k.sA[0], k.sA[1]}, k.ws_g, k.ws_s, k.ws_r, k.Bsz * k.D, k.D, k.K, k.N};
  return launch_carry<true>(c, st);
}

hipError_t launch_bwd_reduce(const BwdK& k, hipStream_t st) {
  hipLaunchKernelGGL(bwd_reduce_bc, dim3(grid_for(k.Bsz * k.G * k.L, 256)), dim3(256), 0, st, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bwd_reduce_params, dim3((unsigned)((k.D * k.N + 63) / 64), 3), dim3(1024), 0,
                     st, k);
  return hipGetLastError();
}

hipError_t launch_fill(float* p, int64_t n, float v, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_f32, dim3(grid_for(n, 256)), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

hipError_t launch_copy4d(const void* src, const int64_t ss[4], const int64_t sdim[4], void* dst,
                         const int64_t ds[4], const int64_t ddim[4], int esize, hipStream_t st) {
  const int64_t total = ddim[0] * ddim[1] * ddim[2] * ddim[3];
  if (total <= 0) return hipSuccess;
  Dims4 a, b, c, d;
  for (int i = 0; i < 4; ++i) {
    a.v[i] = ss[i]; b.v[i] = sdim[i]; c.v[i] = ds[i]; d.v[i] = ddim[i];
  }
  const dim3 grid(grid_for(total, 256));
  if (esize == 4)
    hipLaunchKernelGGL(copy4d<uint32_t>, grid, dim3(256), 0, st, (const uint32_t*)src, a, b,
                       (uint32_t*)dst, c, d);
  else
    hipLaunchKernelGGL(copy4d<uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)src, a, b,
                       (uint16_t*)dst, c, d);
  return hipGetLastError();
}

hipError_t launch_relayout(const void* src, const int64_t s[4], int esize, void* dst,
                           int64_t Bsz, int64_t G, int64_t N, int64_t NP, int64_t L,
                           hipStream_t st) {
  const int64_t total = Bsz * G * L * NP;
  if (total <= 0) return hipSuccess;
  const dim3 grid(grid_for(total, 256));
  if (esize == 4)
    hipLaunchKernelGGL(relayout_bc<uint32_t>, grid, dim3(256), 0, st, (const uint32_t*)src, s[0],
                       s[1], s[2], s[3], (uint32_t*)dst, Bsz, G, N, NP, L);
  else
    hipLaunchKernelGGL(relayout_bc<uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)src, s[0],
                       s[1], s[2], s[3], (uint16_t*)dst, Bsz, G, N, NP, L);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdK& k, int io_dtype, int bc_dtype, hipStream_t st, void* const* ev) {
  switch (io_dtype) {
    case S6_F32: return launch_fwd_io<float>(k, bc_dtype, st, ev);
    case S6_BF16: return launch_fwd_io<bf16>(k, bc_dtype, st, ev);
    default: return launch_fwd_io<f16>(k, bc_dtype, st, ev);
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
