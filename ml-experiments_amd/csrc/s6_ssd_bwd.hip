// Mamba-2 SSD backward, the computation of _mamba_chunk_scan_combined_bwd
// (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/ssd_combined.py:335-452).
// The forward quantities (dt', S, chunk states, entering states H, C B^T) are recomputed by
// the forward's prep kernels.  With G = dy (dout * silu(z) when z is given), per batch b,
// head h and chunk c, and the masks of the forward (mlast: same seq_idx as the chunk's last
// step; mprev: same seq_idx as the step before the chunk; CB carries the pairwise mask):
//
//   ssd_bwd_gate       dy = dout silu(z), dz = dout y silu'(z)            (elementwise)
//   (dstates)          dHl_c = sum_l mprev e^{S_l} G_l C_l^T                  MFMA
//   ssd_state_pass_bwd dst_c = dH_{c+1}; dH_c = scale_c dH_{c+1} + dHl_c; dinit = dH_0;
//                      the S_last gradient sum(dH_{c+1} scale_c H_c)
//   ssd_bwd_dx         T2 = mlast e^{S_last - S_s} B_s dst^T, T1 = sum_{l>=s} CB e^{S_l-S_s} G_l
//                      dx = dt'_s (T1 + T2) + D G_s; ddt'_s = x_s . (T1 + T2); dD parts  MFMA
//   ssd_bwd_rows<4>    dB_s += sum_h mlast dt'_s e^{S_last-S_s} x_s^h dst^h; q_s per head MFMA
//   ssd_bwd_rows<5>    dC_l += sum_h mprev e^{S_l} G_l^h H^h;             u_l per head  MFMA
//   ssd_bwd_dcb        dM = G x^T per head; dCB = sum_h dM e^{S_l-S_s} dt'_s; row / column
//                      sums of W = dM CB e^{S_l-S_s} dt'_s, one block per 64x64 tile   MFMA
//   ssd_bwd_bmm<C|B>   dC += dCB B, dB += dCB^T C                                     MFMA
//   ssd_bwd_dt         dS = u + rowsum(W) - colsum(W) - q (+ the S_last terms at the chunk
//                      end); da = reverse cumsum of dS; ddt = A da + ddt'; through clamp,
//                      softplus and bias; dA, ddt_bias parts
//   ssd_bwd_reduce     dA, ddt_bias, dD in fixed order
//
// Every cross-block sum goes through a partial buffer reduced in fixed order: the backward
// is deterministic (no atomics).
#include "s6_ssd_common.h"

namespace s6 {
namespace {

using namespace ssd;

__device__ inline float wave_sum16(float v) {  // sum over the 16 lanes sharing lane / 16
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

__device__ inline int32_t seq_last_of(const SsdK& k, int64_t b, int64_t c) {
  return seq_at(k, b, min((c + 1) * k.Q, k.L) - 1);
}

// ---- gate ----------------------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(kThreads) ssd_bwd_gate(SsdK k) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= k.Bsz * k.L * k.H * k.P) return;
  const int64_t p = i % k.P;
  int64_t r = i / k.P;
  const int64_t hh = r % k.H;
  r /= k.H;
  const int64_t t = r % k.L, b = r / k.L;
  const float go = Elem<T>::load(k.dout, b * k.sdout[0] + t * k.sdout[1] + hh * k.sdout[2] + p);
  const float zz = Elem<T>::load(k.z, b * k.sz[0] + t * k.sz[1] + hh * k.sz[2] + p);
  const float y = Elem<T>::load(k.out_x, b * k.soutx[0] + t * k.soutx[1] + hh * k.soutx[2] + p);
  const float sg = sigmoidf_(zz);
  Elem<T>::store(k.dyw, i, go * zz * sg);
  Elem<T>::store(k.dz, b * k.sdz[0] + t * k.sdz[1] + hh * k.sdz[2] + p,
                 go * y * sg * fmaf(zz, 1.f - sg, 1.f));
}

// ---- state passing backward ----------------------------------------------------------

constexpr int kSpbPer = 4;  // elements per thread

template <typename T>
__global__ void __launch_bounds__(kThreads) ssd_state_pass_bwd(SsdK k) {
  typedef typename Mma<T>::Raw Raw;
  __shared__ float red[kThreads / kWave];
  const int64_t PN = k.P * k.N;
  const int64_t eb = blockIdx.x, hh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  int64_t e[kSpbPer];
  float dH[kSpbPer];
#pragma unroll
  for (int i = 0; i < kSpbPer; ++i) {
    e[i] = eb * (kThreads * kSpbPer) + tid + i * kThreads;  // PN is a multiple of 1024
    const int64_t p = e[i] / k.N, n = e[i] % k.N;
    dH[i] = (k.dfinal && p < k.Pa && n < k.Na)
                ? k.dfinal[b * k.sdfinal[0] + hh * k.sdfinal[1] + p * k.sdfinal[2] + n * k.sdfinal[3]] : 0.f;
  }
  const Raw* hs = (const Raw*)k.hs;
  Raw* dst = (Raw*)k.dst;
  // the next (earlier) chunk's H and dHl are loaded while this one is processed
  auto ofs = [&](int64_t c) { return ((b * k.K + c) * k.H + hh) * PN; };
  float hn[kSpbPer], gn[kSpbPer];
  auto fetch = [&](int64_t c) {
    if (c < 0) return;
#pragma unroll
    for (int i = 0; i < kSpbPer; ++i) {
      hn[i] = Mma<T>::from_raw(hs[ofs(c) + e[i]]);
      gn[i] = k.dhl[ofs(c) + e[i]];
    }
  };
  fetch(k.K - 1);
  for (int64_t c = k.K - 1; c >= 0; --c) {
    float scale = exp_split(k.dacs[((b * k.H + hh) * k.K + c) * k.Q + k.Q - 1]);
    if (k.has_seq) {
      const int32_t prev = c > 0 ? seq_last_of(k, b, c - 1) : 0;
      if (seq_last_of(k, b, c) != prev) scale = 0.f;
    }
    const int64_t o = ofs(c);
    float hc[kSpbPer], gc[kSpbPer];
#pragma unroll
    for (int i = 0; i < kSpbPer; ++i) { hc[i] = hn[i]; gc[i] = gn[i]; }
    fetch(c - 1);
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < kSpbPer; ++i) {
      dst[o + e[i]] = Mma<T>::to_raw(dH[i]);
      part = fmaf(dH[i], hc[i], part);
      dH[i] = fmaf(scale, dH[i], gc[i]);
    }
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) part += __shfl_xor(part, m);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = part;
    __syncthreads();
    if (tid == 0) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kThreads / kWave; ++w) s += red[w];
      k.ddal[((b * k.H + hh) * k.K + c) * k.nE + eb] = s * scale;
    }
    __syncthreads();
  }
  if (k.dinit) {  // [Bsz, H, Pa, Na]
#pragma unroll
    for (int i = 0; i < kSpbPer; ++i) {
      const int64_t p = e[i] / k.N, n = e[i] % k.N;
      if (p < k.Pa && n < k.Na) k.dinit[((b * k.H + hh) * k.Pa + p) * k.Na + n] = dH[i];
    }
  }
}

// ---- dx, direct dt gradient, dD parts ------------------------------------------------

// Block: 64 rows (steps s) of one chunk and head, 4 waves of 16 rows, all of headdim; the
// layout of the forward's chunk scan.  T2 stages dst through LDS in column stages; T1 runs
// as a software pipeline over stages of SUB MFMA K steps (l >= s): the dy rows and this
// wave's CB column values of stage i + 1 are loaded while stage i computes, dy goes
// transposed into a double LDS buffer, one barrier per stage.  The epilogue stages
// T1 + T2 through LDS so that x, dy and dx move as 16-byte rows.
template <typename T, int P, int N>
__global__ void __launch_bounds__(kThreads) ssd_bwd_dx(SsdK k) {
  typedef Mma<T> M;
  typedef typename M::Raw Raw;
  constexpr int VE = M::kVe;
  constexpr int PT = P / 16;
  constexpr int ES = sizeof(Raw);
  constexpr int SUB = (ES == 2 || P <= 64) ? 2 : 1;       // MFMA K steps per stage
  constexpr int KST = SUB * kKs;                           // steps per stage
  constexpr int LP = KST + 8;                              // LDS row pitch, 16-byte rows
  constexpr int XC = KST * (P / VE);                       // 16-byte dy chunks per stage
  constexpr int XL = (XC + kThreads - 1) / kThreads;
  constexpr int YP = P + 4;                                // T staging pitch (floats)
  constexpr int HCH = N < 128 ? N : ((ES == 4 && P == 128) ? 64 : 128);  // dst columns per stage
  constexpr int HP = HCH + 8;
  constexpr bool TR = ES == 2;                             // row-major dy + transposing reads
  constexpr int GPT = P + 16;                              // row-major dy pitch (TR)
  constexpr int XS_BYTES = TR ? 2 * KST * GPT * ES : 2 * P * LP * ES;
  constexpr int YS_BYTES = 64 * YP * 4, HS_BYTES = P * HP * ES;
  constexpr int SM_A = XS_BYTES > YS_BYTES ? XS_BYTES : YS_BYTES;
  constexpr int SM_BYTES = SM_A > HS_BYTES ? SM_A : HS_BYTES;
  constexpr int RPT = P / VE;                              // threads per row in the epilogue
  __shared__ __attribute__((aligned(16))) char smem[SM_BYTES];
  __shared__ float sls[2][KST];
  __shared__ float dred[kThreads / kWave][P];
  Raw (*gs)[P][LP] = reinterpret_cast<Raw (*)[P][LP]>(smem);
  Raw (*gr_)[KST][GPT] = reinterpret_cast<Raw (*)[KST][GPT]>(smem);
  float (*ys)[YP] = reinterpret_cast<float (*)[YP]>(smem);
  Raw (*dsm)[HP] = reinterpret_cast<Raw (*)[HP]>(smem);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // work id -> (head fastest, row tile, chunk, batch), as the chunk scan
  const int64_t wid = xcd_work_id();
  const int64_t hh = wid % k.H;
  const int lt = (int)((wid / k.H) % (k.Q / 64));
  const int64_t c = (wid / (k.H * (k.Q / 64))) % k.K, b = wid / (k.H * (k.Q / 64) * k.K);
  const int64_t g = hh / k.hpg;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  if (lt * 64 >= lim) return;  // whole block
  const int64_t hrow = ((b * k.H + hh) * k.K + c) * k.Q;
  const float* sq = k.dacs + hrow;
  const float* dq = k.dtq + hrow;
  const int rowbase = lt * 64 + 16 * w;
  const int row = rowbase + (lane & 15);
  const float* cbcol = k.cb + ((b * k.K + c) * k.G + g) * k.Q * k.Q + row;
  const char* gbase = (const char*)k.dy + (b * k.sdy[0] + t0 * k.sdy[1] + hh * k.sdy[2]) * ES;
  const int nst = (lim - lt * 64 + KST - 1) / KST;

  Raw gv[XL][VE];
  float cbv[SUB][8];
  float sv = 0.f;
  auto fetch = [&](int l0) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      const int r = e / (P / VE), col = (e % (P / VE)) * VE;
      if (e < XC && l0 + r < lim) load16<T>(gbase + ((l0 + r) * k.sdy[1] + col) * ES, gv[i]);
      else
#pragma unroll
        for (int q = 0; q < VE; ++q) gv[i][q] = M::to_raw(0.f);
    }
    // in bounds for any l0; steps past the chunk are masked where the value is used (on)
    if (tid < KST) sv = sq[min(l0 + tid, (int)k.Q - 1)];
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks) {
      const bool reach = l0 + ks * kKs + kKs - 1 >= rowbase;  // wave-uniform
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int l = l0 + ks * kKs + M::kidx(lane, j);
        cbv[ks][j] = cbcol[(int64_t)min(l, (int)k.Q - 1) * k.Q];  // masked at use (on)
      }
    }
  };
  fetch(lt * 64);
  // Values used only after the T2 product: loaded here, with the first stage, so that no
  // later step waits a full memory latency for them.
  const float s_last = sq[k.Q - 1];
  // Rows < Q are in bounds; rows past lim are masked where these are used.  Loaded without a
  // condition: a conditional load would wait for itself under its branch.
  const float s_row = sq[row];  // S of this lane's A-operand row
  float s_acc[4];               // S of this lane's accumulator rows
#pragma unroll
  for (int j = 0; j < 4; ++j) s_acc[j] = sq[rowbase + 4 * (lane >> 4) + j];

  f4 acc[PT];
#pragma unroll
  for (int i = 0; i < PT; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

  // T2: B_s dst^T, rows scaled by mlast e^{S_last - S_s}; dst staged through LDS
  {
    // rows past lim read the last valid row (their outputs are scaled by 0 below)
    const Raw* Brow = (const Raw*)k.Bm + b * k.sB[0] + (t0 + min(row, lim - 1)) * k.sB[1] + g * k.sB[2];
    const Raw* D2 = (const Raw*)k.dst + ((b * k.K + c) * k.H + hh) * (int64_t)(P * N);
    constexpr int HC = P * (HCH / VE);
    constexpr int HL = (HC + kThreads - 1) / kThreads;
#pragma unroll
    for (int nc = 0; nc < N; nc += HCH) {
      typename M::Frag af[HCH / kKs];
#pragma unroll
      for (int i = 0; i < HCH / kKs; ++i) af[i] = M::load_row(Brow + nc + i * kKs, lane);
      u4 hv[HL];
#pragma unroll
      for (int i = 0; i < HL; ++i) {
        const int e = tid + i * kThreads;
        const int p = e / (HCH / VE), col = (e % (HCH / VE)) * VE;
        if (e < HC) hv[i] = *reinterpret_cast<const u4*>(D2 + p * N + nc + col);
      }
      if (nc > 0) __syncthreads();
#pragma unroll
      for (int i = 0; i < HL; ++i) {
        const int e = tid + i * kThreads;
        const int p = e / (HCH / VE), col = (e % (HCH / VE)) * VE;
        if (e < HC) *reinterpret_cast<u4*>(&dsm[p][col]) = hv[i];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < HCH / kKs; ++i)
#pragma unroll
        for (int pt = 0; pt < PT; ++pt)
          M::mma(acc[pt], af[i], M::load_row(&dsm[pt * 16 + (lane & 15)][i * kKs], lane));
    }
    __syncthreads();  // dst consumed before the T1 loop writes dy over it
    const int32_t seq_last = k.has_seq ? seq_last_of(k, b, c) : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = rowbase + 4 * (lane >> 4) + j;
      float f = 0.f;
      if (s < lim) {
        f = exp_split(s_last - s_acc[j]);
        if (k.has_seq && seq_at(k, b, t0 + s) != seq_last) f = 0.f;
      }
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) acc[pt][j] *= f;
    }
  }

  // T1: sum_{l >= s} CB[l, s] e^{S_l - S_s} G_l
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    const int l0 = lt * 64 + st * KST;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      if (e < XC) {
        const int r = e / (P / VE), col = (e % (P / VE)) * VE;
        if constexpr (TR) {
          *reinterpret_cast<u4*>(&gr_[buf][r][col]) = *reinterpret_cast<const u4*>(gv[i]);
        } else {
#pragma unroll
          for (int q = 0; q < VE; ++q) gs[buf][col + q][r] = gv[i][q];
        }
      }
    }
    if (tid < KST) sls[buf][tid] = sv;
    float cbc[SUB][8];
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) cbc[ks][j] = cbv[ks][j];
    __syncthreads();
    if (st + 1 < nst) fetch(l0 + KST);
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks) {
      if (l0 + ks * kKs + kKs - 1 >= rowbase) {  // wave-uniform: the slice reaches this wave's rows
        float m[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int li = ks * kKs + M::kidx(lane, j);
          const int l = l0 + li;
          const bool on = l >= row && l < lim && row < lim;
          const float v = cbc[ks][j] * exp_split(sls[buf][li] - s_row);
          m[j] = on ? v : 0.f;
        }
        const typename M::Frag a = M::from_float(m);
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
          if constexpr (TR) M::mma(acc[pt], a, M::load_tr(&gr_[buf][ks * kKs][pt * 16], GPT, lane));
          else M::mma(acc[pt], a, M::load_row(&gs[buf][pt * 16 + (lane & 15)][ks * kKs], lane));
        }
      }
    }
  }

  // epilogue through LDS: dx = dt'_s (T1 + T2) + D G_s, ddt'_s = x_s . (T1 + T2), dD partial
  __syncthreads();  // every wave is done reading dy from the buffer ys reuses
#pragma unroll
  for (int pt = 0; pt < PT; ++pt)
#pragma unroll
    for (int j = 0; j < 4; ++j) ys[16 * w + 4 * (lane >> 4) + j][pt * 16 + (lane & 15)] = acc[pt][j];
  __syncthreads();
  const char* xbase = (const char*)k.x + (b * k.sx[0] + t0 * k.sx[1] + hh * k.sx[2]) * ES;
  const int col = (tid % RPT) * VE;  // fixed per thread: kThreads is a multiple of RPT
  float dd[VE];
#pragma unroll
  for (int q = 0; q < VE; ++q) dd[q] = 0.f;
  float Dv[VE];
#pragma unroll
  for (int q = 0; q < VE; ++q)
    Dv[q] = !k.has_D ? 0.f : !k.D_hdim ? k.Dp[hh * k.sD[0]]
            : col + q < k.Pa ? k.Dp[hh * k.sD[0] + (col + q) * k.sD[1]] : 0.f;
  for (int e = tid; e < 64 * RPT; e += kThreads) {  // uniform trip count over the block
    const int r = e / RPT;
    const int s = lt * 64 + r;
    const bool valid = s < lim;
    Raw xr[VE], gr[VE];
    if (valid) {
      load16<T>(xbase + (s * k.sx[1] + col) * ES, xr);
      load16<T>(gbase + (s * k.sdy[1] + col) * ES, gr);
    } else {
#pragma unroll
      for (int q = 0; q < VE; ++q) xr[q] = gr[q] = M::to_raw(0.f);
    }
    const float dts = valid ? dq[s] : 0.f;
    float xsum = 0.f;
    Raw o[VE];
#pragma unroll
    for (int q = 0; q < VE; ++q) {
      const float a = ys[r][col + q];
      const float xv = M::from_raw(xr[q]), gvv = M::from_raw(gr[q]);
      xsum = fmaf(xv, a, xsum);
      dd[q] = fmaf(gvv, xv, dd[q]);
      o[q] = M::to_raw(fmaf(Dv[q], gvv, dts * a));
    }
    if (valid)
      *reinterpret_cast<u4*>((char*)k.dx + (b * k.sdx[0] + (t0 + s) * k.sdx[1] + hh * k.sdx[2] + col) * ES) =
          *reinterpret_cast<const u4*>(o);
#pragma unroll
    for (int m = 1; m < RPT; m <<= 1) xsum += __shfl_xor(xsum, m);  // the row's RPT lanes are adjacent
    if ((tid % RPT) == 0 && valid) k.ddtd[hrow + s] = xsum;
  }
  if (k.has_D) {
    // sum dd over the threads holding the same columns: lanes that differ in bits >= log2(RPT)
#pragma unroll
    for (int q = 0; q < VE; ++q) {
      float v = dd[q];
#pragma unroll
      for (int m = RPT; m < kWave; m <<= 1) v += __shfl_xor(v, m);
      dd[q] = v;
    }
    if (lane < RPT)
#pragma unroll
      for (int q = 0; q < VE; ++q) dred[w][col + q] = dd[q];
    __syncthreads();
    const int64_t brow = (b * k.K + c) * (k.Q / 64) + lt;
    if (k.D_hdim) {
      for (int p = tid; p < P; p += kThreads)
        k.dDp[(brow * k.H + hh) * P + p] = dred[0][p] + dred[1][p] + dred[2][p] + dred[3][p];
    } else if (tid < kWave) {
      float v = 0.f;
      for (int p = tid; p < P; p += kWave) v += dred[0][p] + dred[1][p] + dred[2][p] + dred[3][p];
#pragma unroll
      for (int m = 1; m < kWave; m <<= 1) v += __shfl_xor(v, m);
      if (tid == 0) k.dDp[brow * k.H + hh] = v;
    }
  }
}

// ---- per-group row products: dB from the chunk states (MODE 4), dC from the entering
// states (MODE 5) ------------------------------------------------------------------------

// Block: 64 rows of one chunk and group and a slice of NC dstate columns; it loops over the
// group's heads, accumulating f_h(l) A_h[l, :] mat_h[:, n] (A = x, mat = dst for dB; A = dy,
// mat = H for dC) and writing the per-head row sums against B (C) as one partial per column
// slice.  The next head's matrix slice, A fragments and cumsums are loaded while the current
// head computes; the matrix goes transposed (dstate-major, K = headdim contiguous) into a
// double LDS buffer written with lanes along headdim, so the 2-byte writes do not collide.
// Occupancy target of 4 waves per SIMD for MODE 5 at headdim 64 x dstate 128 with 16-bit
// inputs, which fits it in 121 registers without spilling (the compiler's own layout takes
// 144, 3 waves); MODE 4 and fp32 inputs would spill at that budget and keep the default.
template <typename T, int P, int N, int MODE>
__global__ void __launch_bounds__(kThreads)
    __attribute__((amdgpu_waves_per_eu((MODE == 5 && P == 64 && N == 128 && sizeof(T) == 2) ? 4 : 1)))
    ssd_bwd_rows(SsdK k) {
  typedef Mma<T> M;
  typedef typename M::Raw Raw;
  typedef typename M::Frag Frag;
  constexpr int VE = M::kVe;
  constexpr int ES = sizeof(Raw);
  constexpr int NC = N < 64 ? N : 64;       // dstate columns per block
  constexpr int NS = N / NC;
  constexpr int NT = NC / 16;
  constexpr int MP = P + 8;                 // LDS pitch, 16-byte rows (transposed, fp32)
  constexpr bool TR = ES == 2;              // 16-bit: row-major slice + transposing reads
  constexpr int RPT_ = NC + 16;             // row-major pitch (TR)
  constexpr int BUF_BYTES = TR ? P * RPT_ * ES : NC * MP * ES;
  constexpr int NB = 2 * BUF_BYTES <= 40960 ? 2 : 1;
  constexpr int MC = P * (NC / VE);         // 16-byte chunks of one head's matrix slice
  constexpr int ML = (MC + kThreads - 1) / kThreads;
  constexpr int KF = P / kKs;
  __shared__ __attribute__((aligned(16))) char smem[NB * BUF_BYTES];
  Raw (*ms)[NC][MP] = reinterpret_cast<Raw (*)[NC][MP]>(smem);
  Raw (*mr)[P][RPT_] = reinterpret_cast<Raw (*)[P][RPT_]>(smem);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int QT = (int)(k.Q / 64);
  const int64_t wid = xcd_work_id();  // (column slice fastest, row tile, chunk, batch * group)
  const int ns = (int)(wid % NS);
  const int lt = (int)((wid / NS) % QT);
  const int64_t c = (wid / (NS * QT)) % k.K, bg = wid / (NS * QT * k.K);
  const int64_t b = bg / k.G, g = bg % k.G;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  if (lt * 64 >= lim) return;
  const int rowbase = lt * 64 + 16 * w;
  const int row = rowbase + (lane & 15);
  const int64_t* sa = MODE == 4 ? k.sx : k.sdy;
  // A-operand rows past lim read the last valid row: their accumulator rows get f = 0
  const Raw* abase = (const Raw*)(MODE == 4 ? k.x : k.dy) + b * sa[0] + (t0 + min(row, lim - 1)) * sa[1];
  const void* side = MODE == 4 ? k.Bm : k.Cm;
  const int64_t* ss = MODE == 4 ? k.sB : k.sC;
  const int32_t seq_ref = !k.has_seq ? 0
                          : MODE == 4 ? seq_last_of(k, b, c) : (c > 0 ? seq_at(k, b, t0 - 1) : 0);
  const int64_t nrs = k.Bsz * k.H * k.K * k.Q;
  // head-independent: row masks and B (C) at this lane's accumulator positions
  bool rv[4];
  float sd[4][NT];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int l = rowbase + 4 * (lane >> 4) + j;
    rv[j] = l < lim && (!k.has_seq || seq_at(k, b, t0 + l) == seq_ref);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      // rows past lim read the last valid row: their terms are scaled by f = 0 (rv)
      sd[j][nt] = Elem<T>::load(side, b * ss[0] + (t0 + min(l, lim - 1)) * ss[1] + g * ss[2] + ns * NC + nt * 16 + (lane & 15));
  }
  f4 tot[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) tot[i] = f4{0.f, 0.f, 0.f, 0.f};

  Raw mv[ML][VE];
  Frag af[KF];
  float sqv[4], dqv[4], slv = 0.f;
  auto fetch = [&](int64_t hh) {
    const Raw* mat = (const Raw*)(MODE == 4 ? k.dst : k.hs) + ((b * k.K + c) * k.H + hh) * (int64_t)(P * N);
#pragma unroll
    for (int i = 0; i < ML; ++i) {
      const int e = tid + i * kThreads;
      const int p = TR ? e / (NC / VE) : e % P, n0 = TR ? (e % (NC / VE)) * VE : (e / P) * VE;
      if (e < MC) load16<T>(mat + p * N + ns * NC + n0, mv[i]);
    }
#pragma unroll
    for (int kk = 0; kk < KF; ++kk) af[kk] = M::load_row(abase + hh * sa[2] + kk * kKs, lane);
    const int64_t hrow = ((b * k.H + hh) * k.K + c) * k.Q;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = rowbase + 4 * (lane >> 4) + j;
      sqv[j] = k.dacs[hrow + l];  // l < Q: in bounds; rows past lim get f = 0 (rv)
      dqv[j] = MODE == 4 ? k.dtq[hrow + l] : 0.f;
    }
    if (MODE == 4) slv = k.dacs[hrow + k.Q - 1];
  };

  const int64_t h0 = g * k.hpg;
  fetch(h0);
  for (int hi = 0; hi < (int)k.hpg; ++hi) {
    const int buf = NB == 2 ? (hi & 1) : 0;
    const int64_t hh = h0 + hi;
    if (NB == 1 && hi > 0) __syncthreads();  // the single buffer is consumed
#pragma unroll
    for (int i = 0; i < ML; ++i) {
      const int e = tid + i * kThreads;
      if (e < MC) {
        if constexpr (TR) {
          const int p = e / (NC / VE), n0 = (e % (NC / VE)) * VE;
          *reinterpret_cast<u4*>(&mr[buf][p][n0]) = *reinterpret_cast<const u4*>(mv[i]);
        } else {
          const int p = e % P, n0 = (e / P) * VE;
#pragma unroll
          for (int q = 0; q < VE; ++q) ms[buf][n0 + q][p] = mv[i][q];
        }
      }
    }
    Frag ac[KF];
    float sqc[4], dqc[4];
#pragma unroll
    for (int kk = 0; kk < KF; ++kk) ac[kk] = af[kk];
#pragma unroll
    for (int j = 0; j < 4; ++j) { sqc[j] = sqv[j]; dqc[j] = dqv[j]; }
    const float slc = slv;
    __syncthreads();
    if (hi + 1 < (int)k.hpg) fetch(hh + 1);
    f4 acc[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KF; ++kk)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if constexpr (TR) M::mma(acc[nt], ac[kk], M::load_tr(&mr[buf][kk * kKs][nt * 16], RPT_, lane));
        else M::mma(acc[nt], ac[kk], M::load_row(&ms[buf][nt * 16 + (lane & 15)][kk * kKs], lane));
      }
    const int64_t hrow = ((b * k.H + hh) * k.K + c) * k.Q;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = rowbase + 4 * (lane >> 4) + j;
      const float f = !rv[j] ? 0.f : MODE == 4 ? dqc[j] * exp_split(slc - sqc[j]) : exp_split(sqc[j]);
      float sv = 0.f;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float a = acc[nt][j] * f;
        sv = fmaf(sd[j][nt], a, sv);
        tot[nt][j] += a;
      }
      sv = wave_sum16(sv);
      if ((lane & 15) == 0 && l < lim) (MODE == 4 ? k.qv : k.uv)[ns * nrs + hrow + l] = sv;
    }
  }
  float* outp = MODE == 4 ? k.dBp : k.dCp;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int l = rowbase + 4 * (lane >> 4) + j;
    if (l >= lim) continue;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      outp[((b * k.L + t0 + l) * k.G + g) * N + ns * NC + nt * 16 + (lane & 15)] = tot[nt][j];
  }
}

// ---- dCB and the intra-chunk decay terms ---------------------------------------------

// Block: one 64x64 tile (I, J), J <= I, of dCB for one chunk and group; it loops over the
// group's heads.  Per head, dM = G_I X_J^T on MFMA, with the x tile staged untransposed in
// LDS (its rows are the B operand's K-contiguous rows) and each wave's dy rows straight from
// global memory; then, elementwise, dCB += dM e^{S_l - S_s} dt'_s and W = that times CB, whose
// row sums (per tile J: partials summed by ssd_bwd_dt) and column sums (reduced over the
// block's waves in LDS) feed the dt gradient.  The next head's x tile, dy fragments and
// cumsums are loaded while the current head computes; CB's values at this lane's
// accumulator positions do not depend on the head and stay in registers.
template <typename T, int P>
__global__ void __launch_bounds__(kThreads) ssd_bwd_dcb(SsdK k) {
  typedef Mma<T> M;
  typedef typename M::Raw Raw;
  typedef typename M::Frag Frag;
  constexpr int VE = M::kVe;
  constexpr int XP = P + 8;                 // x tile pitch, 16-byte rows
  constexpr int XC = 64 * (P / VE);         // 16-byte chunks per x tile
  constexpr int XL = (XC + kThreads - 1) / kThreads;
  constexpr int KF = P / kKs;               // MFMA K steps over headdim
  __shared__ __attribute__((aligned(16))) Raw xs[2][64][XP];
  __shared__ float csred[2][kThreads / kWave][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int QT = (int)(k.Q / 64);
  const int64_t ntile = QT * (QT + 1) / 2;
  const int64_t wid = xcd_work_id();  // (tile fastest, chunk, batch * group)
  int I = 0, J = (int)(wid % ntile);
  while (J > I) { J -= I + 1; ++I; }
  const int64_t c = (wid / ntile) % k.K, bg = wid / (ntile * k.K);
  const int64_t b = bg / k.G, g = bg % k.G;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  if (I * 64 >= lim) return;  // whole block (J <= I)
  const int rowbase = I * 64 + 16 * w;
  const int row = rowbase + (lane & 15);
  const float* cbm = k.cb + ((b * k.K + c) * k.G + g) * k.Q * k.Q;
  const int64_t nrs = k.Bsz * k.H * k.K * k.Q;  // elements of one row-sum partial
  float cbv[4][4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = rowbase + 4 * (lane >> 4) + j, s = J * 64 + ct * 16 + (lane & 15);
      cbv[ct][j] = cbm[(int64_t)l * k.Q + s];  // l, s < Q: in bounds; used only where on
    }
  f4 dcb[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) dcb[ct] = f4{0.f, 0.f, 0.f, 0.f};

  Raw xv[XL][VE];
  Frag gf[KF];
  float slv[4], ssv[4], dsv[4];
  auto fetch = [&](int64_t hh) {
    const char* xb = (const char*)k.x + (b * k.sx[0] + t0 * k.sx[1] + hh * k.sx[2]) * sizeof(Raw);
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      const int r = e / (P / VE), col = (e % (P / VE)) * VE;
      const int s = J * 64 + r;
      if (e < XC && s < lim) load16<T>(xb + (s * k.sx[1] + col) * sizeof(Raw), xv[i]);
      else
#pragma unroll
        for (int q = 0; q < VE; ++q) xv[i][q] = M::to_raw(0.f);
    }
    // rows past lim read the last valid row: every dM term of such a row is masked below
    const Raw* grow = (const Raw*)k.dy + b * k.sdy[0] + (t0 + min(row, lim - 1)) * k.sdy[1] + hh * k.sdy[2];
#pragma unroll
    for (int kk = 0; kk < KF; ++kk) gf[kk] = M::load_row(grow + kk * kKs, lane);
    const int64_t hrow = ((b * k.H + hh) * k.K + c) * k.Q;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = rowbase + 4 * (lane >> 4) + j;
      slv[j] = k.dacs[hrow + l];  // l < Q: in bounds; used only where on
    }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int s = J * 64 + ct * 16 + (lane & 15);  // < Q: rows past lim hold dt' = 0
      ssv[ct] = k.dacs[hrow + s];
      dsv[ct] = k.dtq[hrow + s];
    }
  };
  auto write_csp = [&](int64_t hh, int buf) {
    k.csp[(((b * k.H + hh) * k.K + c) * QT + I) * k.Q + J * 64 + tid] =
        csred[buf][0][tid] + csred[buf][1][tid] + csred[buf][2][tid] + csred[buf][3][tid];
  };

  const int64_t h0 = g * k.hpg;
  fetch(h0);
  for (int hi = 0; hi < (int)k.hpg; ++hi) {
    const int buf = hi & 1;
    const int64_t hh = h0 + hi;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      if (e < XC) {
        const int r = e / (P / VE), col = (e % (P / VE)) * VE;
        *reinterpret_cast<u4*>(&xs[buf][r][col]) = *reinterpret_cast<const u4*>(xv[i]);
      }
    }
    Frag gc[KF];
    float slc[4], ssc[4], dsc[4];
#pragma unroll
    for (int kk = 0; kk < KF; ++kk) gc[kk] = gf[kk];
#pragma unroll
    for (int j = 0; j < 4; ++j) { slc[j] = slv[j]; ssc[j] = ssv[j]; dsc[j] = dsv[j]; }
    __syncthreads();
    if (hi > 0 && tid < 64) write_csp(hh - 1, buf ^ 1);
    if (hi + 1 < (int)k.hpg) fetch(hh + 1);
    f4 dM[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) dM[ct] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KF; ++kk)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        M::mma(dM[ct], gc[kk], M::load_row(&xs[buf][ct * 16 + (lane & 15)][kk * kKs], lane));
    float rsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int s = J * 64 + ct * 16 + (lane & 15);
      float colsum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int l = rowbase + 4 * (lane >> 4) + j;
        const bool on = s <= l && l < lim && s < lim;
        const float dme = on ? dM[ct][j] * exp_split(slc[j] - ssc[ct]) * dsc[ct] : 0.f;
        dcb[ct][j] += dme;
        const float wv = dme * cbv[ct][j];
        rsum[j] += wv;
        colsum += wv;
      }
      colsum += __shfl_xor(colsum, 16);
      colsum += __shfl_xor(colsum, 32);
      if (lane < 16) csred[buf][w][ct * 16 + lane] = colsum;
    }
    const int64_t hrow = ((b * k.H + hh) * k.K + c) * k.Q;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = rowbase + 4 * (lane >> 4) + j;
      const float v = wave_sum16(rsum[j]);
      if ((lane & 15) == 0 && l < lim) k.rs[J * nrs + hrow + l] = v;
    }
  }
  __syncthreads();
  if (tid < 64) write_csp(h0 + k.hpg - 1, (int)((k.hpg - 1) & 1));

  float* out = k.dcb + ((b * k.K + c) * k.G + g) * k.Q * k.Q;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = rowbase + 4 * (lane >> 4) + j;
      const int s = J * 64 + ct * 16 + (lane & 15);
      float v = dcb[ct][j];
      if (!(l < lim && s < lim)) v = 0.f;
      else if (k.has_seq && seq_at(k, b, t0 + l) != seq_at(k, b, t0 + s)) v = 0.f;
      out[(int64_t)l * k.Q + s] = v;
    }
  }
}

// ---- dC += dCB B (MODE 0), dB += dCB^T C (MODE 1) -------------------------------------

template <typename T, int N, int MODE>
__global__ void __launch_bounds__(kThreads) ssd_bwd_bmm(SsdK k) {
  typedef Mma<T> M;
  typedef typename M::Raw Raw;
  constexpr int VE = M::kVe;
  constexpr int NT = N / 16;
  constexpr int ES = sizeof(Raw);
  constexpr bool TR = ES == 2;  // 16-bit: row-major slice + transposing reads
  constexpr int OPT = N + 16;
  constexpr int OS_BYTES = TR ? kKs * OPT * ES : N * kLp * ES;
  __shared__ __attribute__((aligned(16))) char smem[OS_BYTES];
  Raw (*os)[kLp] = reinterpret_cast<Raw (*)[kLp]>(smem);
  Raw (*orr)[OPT] = reinterpret_cast<Raw (*)[OPT]>(smem);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t wid = xcd_work_id();  // (row tile fastest, chunk, batch * group)
  const int lt = (int)(wid % (k.Q / 64));
  const int64_t c = (wid / (k.Q / 64)) % k.K, b = wid / ((k.Q / 64) * k.K * k.G), g = (wid / ((k.Q / 64) * k.K)) % k.G;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  if (lt * 64 >= lim) return;
  const int rowbase = lt * 64 + 16 * w;
  const int row = rowbase + (lane & 15);
  const float* dcbm = k.dcb + ((b * k.K + c) * k.G + g) * k.Q * k.Q;
  const int64_t* so = MODE == 0 ? k.sB : k.sC;  // the staged operand: B for dC, C for dB
  const char* obase = (const char*)(MODE == 0 ? k.Bm : k.Cm) + (b * so[0] + t0 * so[1] + g * so[2]) * ES;
  f4 acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};
  const int k0 = MODE == 0 ? 0 : lt * 64;
  const int k1 = MODE == 0 ? min(lt * 64 + 64, lim) : lim;
  for (int s0 = k0; s0 < k1; s0 += kKs) {
    __syncthreads();
    for (int e = tid; e < kKs * (N / VE); e += kThreads) {
      const int r = e / (N / VE), col = (e % (N / VE)) * VE;
      Raw v[VE];
      if (s0 + r < lim) load16<T>(obase + ((s0 + r) * so[1] + col) * ES, v);
      else
#pragma unroll
        for (int q = 0; q < VE; ++q) v[q] = M::to_raw(0.f);
      if constexpr (TR) {
        *reinterpret_cast<u4*>(&orr[r][col]) = *reinterpret_cast<const u4*>(v);
      } else {
#pragma unroll
        for (int q = 0; q < VE; ++q) os[col + q][r] = v[q];
      }
    }
    __syncthreads();
    const bool reach = MODE == 0 ? s0 <= rowbase + 15 : s0 + kKs - 1 >= rowbase;  // wave-uniform
    if (reach) {
      float m[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kk = s0 + M::kidx(lane, j);
        const bool on = row < lim && kk < lim && (MODE == 0 ? kk <= row : kk >= row);
        const float v = MODE == 0 ? dcbm[(int64_t)row * k.Q + kk] : dcbm[(int64_t)kk * k.Q + row];
        m[j] = on ? v : 0.f;
      }
      const typename M::Frag a = M::from_float(m);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if constexpr (TR) M::mma(acc[nt], a, M::load_tr(&orr[0][nt * 16], OPT, lane));
        else M::mma(acc[nt], a, M::load_row(&os[nt * 16 + (lane & 15)][0], lane));
      }
    }
  }
  const float* part = MODE == 0 ? k.dCp : k.dBp;
  void* outp = MODE == 0 ? k.dCo : k.dBo;
  const int64_t* sop = MODE == 0 ? k.sdCo : k.sdBo;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int l = rowbase + 4 * (lane >> 4) + j;
    if (l >= lim) continue;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = nt * 16 + (lane & 15);
      if (n >= k.Na) continue;  // padded dstate column
      const float v = acc[nt][j] + part[((b * k.L + t0 + l) * k.G + g) * N + n];
      Elem<T>::store(outp, b * sop[0] + (t0 + l) * sop[1] + g * sop[2] + n, v);
    }
  }
}

// ---- dt, dA, ddt_bias ----------------------------------------------------------------

// One wave per (batch, head, chunk): lane i holds steps 4i .. 4i+3.  da_j = sum_{k >= j} dS_k
// is a suffix scan: per-lane suffix sums plus a wave scan of the lane totals from the top.
__global__ void __launch_bounds__(kWave) ssd_bwd_dt(SsdK k) {
  const int lane = threadIdx.x;
  const int64_t c = blockIdx.x, hh = blockIdx.y, b = blockIdx.z;
  const int64_t hrow = ((b * k.H + hh) * k.K + c) * k.Q;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  const int QT = (int)(k.Q / 64);
  const int nI = (lim + 63) / 64;  // row tiles that ran
  const int64_t nrs = k.Bsz * k.H * k.K * k.Q;
  float ddal = 0.f;
  for (int64_t e = lane; e < k.nE; e += kWave) ddal += k.ddal[((b * k.H + hh) * k.K + c) * k.nE + e];
  float qv[4], dS[4];
  float qsum = 0.f;
  const int nsl = (int)(k.N / (k.N < 64 ? k.N : 64));  // dstate column slices of ssd_bwd_rows
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = 4 * lane + q;
    qv[q] = 0.f;
    if (j < lim)
      for (int i = 0; i < nsl; ++i) qv[q] += k.qv[i * nrs + hrow + j];
    qsum += qv[q];
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    qsum += __shfl_xor(qsum, m);
    ddal += __shfl_xor(ddal, m);
  }
  float tot = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = 4 * lane + q;
    float d = j == k.Q - 1 ? ddal + qsum : 0.f;
    if (j < lim) {
      float cs = 0.f;
      for (int I = j / 64; I < nI; ++I) cs += k.csp[(((b * k.H + hh) * k.K + c) * QT + I) * k.Q + j];
      float rsj = 0.f;  // row sum: one partial per column tile J <= j / 64
      for (int J = 0; J <= j / 64; ++J) rsj += k.rs[J * nrs + hrow + j];
      float uvj = 0.f;
      for (int i = 0; i < nsl; ++i) uvj += k.uv[i * nrs + hrow + j];
      d += uvj + rsj - cs - qv[q];
    }
    dS[q] = d;
    tot += d;
  }
  float incl = tot;  // inclusive scan of lane totals from the last lane down
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float u = __shfl_down(incl, m);
    if (lane + m < kWave) incl += u;
  }
  float da = incl - tot;  // sum over the lanes above
  const float A = k.A[hh * k.sA];
  const float bias = k.has_bias ? k.bias[hh * k.sbias] : 0.f;
  float dAacc = 0.f, dbacc = 0.f;
#pragma unroll
  for (int q = 3; q >= 0; --q) {
    const int j = 4 * lane + q;
    da += dS[q];
    if (j < lim) {
      const float dtp = k.dtq[hrow + j];
      float g = fmaf(A, da, k.ddtd[hrow + j]);
      dAacc = fmaf(dtp, da, dAacc);
      const float v = load_any(k.dt, b * k.sdt[0] + (t0 + j) * k.sdt[1] + hh * k.sdt[2], k.io) + bias;
      const float sp = k.softplus ? softplus20(v) : v;
      if (sp < k.dt_min || sp > k.dt_max) g = 0.f;
      if (k.softplus && v <= 20.f) g *= sigmoidf_(v);
      store_any(k.ddt, b * k.sddt[0] + (t0 + j) * k.sddt[1] + hh * k.sddt[2], g, k.io);
      dbacc += g;
    }
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    dAacc += __shfl_xor(dAacc, m);
    dbacc += __shfl_xor(dbacc, m);
  }
  if (lane == 0) {
    k.dAp[(b * k.K + c) * k.H + hh] = dAacc;
    k.dbp[(b * k.K + c) * k.H + hh] = dbacc;
  }
}

// One wave per output (dA[h], ddt_bias[h], dD[h(, p)]): lanes take every 64th partial row,
// then a fixed-order wave sum.
__global__ void __launch_bounds__(kWave) ssd_bwd_reduce(SsdK k) {
  const int lane = threadIdx.x;
  const int64_t o = blockIdx.x;
  const int64_t rows = k.Bsz * k.K;
  float s = 0.f;
  if (o < 2 * k.H) {
    const float* src = o < k.H ? k.dAp : k.dbp;
    const int64_t h = o % k.H;
    for (int64_t r = lane; r < rows; r += kWave) s += src[r * k.H + h];
  } else {
    const int64_t i = o - 2 * k.H;
    const int64_t nd = k.D_hdim ? k.H * k.P : k.H;
    const int64_t qt = k.Q / 64;
    for (int64_t r = lane; r < rows * qt; r += kWave) {
      const int64_t lt = r % qt, c = (r / qt) % k.K;
      if (lt * 64 >= min(k.Q, k.L - c * k.Q)) continue;  // tile past the sequence end: no partial
      s += k.dDp[r * nd + i];
    }
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) s += __shfl_xor(s, m);
  if (lane != 0) return;
  if (o < k.H) k.dA[o] = s;
  else if (o < 2 * k.H) { if (k.ddt_bias) k.ddt_bias[o - k.H] = s; }
  else if (!k.D_hdim) k.dD[o - 2 * k.H] = s;
  else {  // [H, Pa]
    const int64_t i = o - 2 * k.H, p = i % k.P;
    if (p < k.Pa) k.dD[(i / k.P) * k.Pa + p] = s;
  }
}

// ---- dispatch ------------------------------------------------------------------------

template <typename T, int P, int N>
hipError_t ssd_bwd_pn(const SsdK& k, hipStream_t st) {
  hipError_t e;
  const unsigned qt = (unsigned)(k.Q / 64);
  const dim3 blk(kThreads);
  if (k.has_z) {
    const int64_t n = k.Bsz * k.L * k.H * k.P;
    hipLaunchKernelGGL((ssd_bwd_gate<T>), dim3((unsigned)((n + kThreads - 1) / kThreads)), blk, 0, st, k);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if ((e = launch_ssd_dstates(k, st)) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_state_pass_bwd<T>), dim3((unsigned)k.nE, (unsigned)k.H, (unsigned)k.Bsz), blk, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_dx<T, P, N>), dim3((unsigned)(qt * k.K * k.Bsz * k.H)), blk, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_rows<T, P, N, 4>), dim3((unsigned)(N / (N < 64 ? N : 64) * qt * k.K * k.Bsz * k.G)), blk, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_rows<T, P, N, 5>), dim3((unsigned)(N / (N < 64 ? N : 64) * qt * k.K * k.Bsz * k.G)), blk, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_dcb<T, P>), dim3((unsigned)(qt * (qt + 1) / 2 * k.K * k.Bsz * k.G)), blk, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_bmm<T, N, 0>), dim3((unsigned)(qt * k.K * k.Bsz * k.G)), blk, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_bmm<T, N, 1>), dim3((unsigned)(qt * k.K * k.Bsz * k.G)), blk, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_bwd_dt), dim3((unsigned)k.K, (unsigned)k.H, (unsigned)k.Bsz), dim3(kWave), 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int64_t nout = 2 * k.H + (k.has_D ? (k.D_hdim ? k.H * k.P : k.H) : 0);
  hipLaunchKernelGGL((ssd_bwd_reduce), dim3((unsigned)nout), dim3(kWave), 0, st, k);
  return hipGetLastError();
}

template <typename T, int P>
hipError_t ssd_bwd_p(const SsdK& k, hipStream_t st) {
  switch (k.N) {
    case 32: return ssd_bwd_pn<T, P, 32>(k, st);
    case 64: return ssd_bwd_pn<T, P, 64>(k, st);
    case 128: return ssd_bwd_pn<T, P, 128>(k, st);
    case 256: return ssd_bwd_pn<T, P, 256>(k, st);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
hipError_t ssd_bwd_t(const SsdK& k, hipStream_t st) {
  switch (k.P) {
    case 32: return ssd_bwd_p<T, 32>(k, st);
    case 64: return ssd_bwd_p<T, 64>(k, st);
    case 128: return ssd_bwd_p<T, 128>(k, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_ssd_bwd(const SsdK& k, hipStream_t st) {
  hipError_t e = launch_ssd_prep(k, st);
  if (e != hipSuccess) return e;
  if (k.io == S6_BF16) return ssd_bwd_t<bf16>(k, st);
  if (k.io == S6_F16) return ssd_bwd_t<f16>(k, st);
  if (k.io == S6_F32) return ssd_bwd_t<float>(k, st);
  return hipErrorInvalidValue;
}

}  // namespace s6
