// Mamba-2 SSD forward (chunked scan with scalar A per head), the computation of
// _mamba_chunk_scan_combined_fwd (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/
// triton/ssd_combined.py:281-332), in five kernels:
//
//   ssd_cumsum        dt -> dt' = clamp(softplus(dt + bias)), S = cumsum(dt' A) per chunk
//                     (a wave scan per chunk and head)
//                     (ssd_chunk_state.py:34-84 semantics)
//   ssd_chunk_state   st_c[p, n] = sum_l x_l[p] (dt'_l e^{S_last - S_l}) B_l[n]     MFMA
//                     (ssd_chunk_state.py:177-266)
//   ssd_state_pass    H_{c+1} = e^{S_last,c} H_c + st_c, reset across seq_idx changes
//                     (ssd_state_passing.py:28-91)
//   ssd_bmm           CB_c[l, s] = C_l . B_s within each chunk, lower triangle        MFMA
//                     (ssd_bmm.py:35-106)
//   ssd_chunk_scan    y_l = e^{S_l} C_l H_c^T + sum_{s<=l} CB[l,s] e^{S_l-S_s} dt'_s x_s
//                     + D x_l, then * silu(z)                                       MFMA
//                     (ssd_chunk_scan.py:43-185)
//
// MFMA operands (layout in s6_ssd_common.h): operands whose K axis is the sequence (x and B in the chunk state, x in the
// chunk scan) are staged through LDS transposed, so each lane's 8 K-items are one 16-byte
// LDS read; operands whose K axis is dstate (C, B in CB; C and the passed states in the
// scan) are read straight from global memory, 16 bytes per lane.
//
// Precision follows the reference's rounding points: the scaled B of the chunk state and
// the decayed CB of the chunk scan are rounded to the input type before the MFMA, the
// passed states are stored in the input type, chunk states, CB and all accumulation are
// fp32.
#include "s6_ssd_common.h"

namespace s6 {
namespace {

using namespace ssd;

// ---- 1. dt processing and per-chunk cumulative decay ---------------------------------

// One wave per (batch, chunk, head): lane i holds steps 4i .. 4i+3 (chunk <= 256), sums
// them, and an inclusive wave scan of the lane totals gives each lane its prefix.
__global__ void __launch_bounds__(kWave) ssd_cumsum(SsdK k) {
  const int lane = threadIdx.x;
  const int64_t c = blockIdx.x, hh = blockIdx.y, b = blockIdx.z;
  const float A = k.A[hh * k.sA];
  const float bias = k.has_bias ? k.bias[hh * k.sbias] : 0.f;
  const int64_t row = ((b * k.H + hh) * k.K + c) * k.Q;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  float v[4], a[4];
  float tot = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int l = 4 * lane + q;
    v[q] = 0.f;
    if (l < lim) {
      v[q] = load_any(k.dt, b * k.sdt[0] + (t0 + l) * k.sdt[1] + hh * k.sdt[2], k.io) + bias;
      if (k.softplus) v[q] = softplus20(v[q]);
      v[q] = fminf(fmaxf(v[q], k.dt_min), k.dt_max);
    }
    tot += v[q] * A;
    a[q] = tot;
  }
  float incl = tot;  // inclusive scan of the lane totals
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float u = __shfl_up(incl, m);
    if (lane >= m) incl += u;
  }
  const float pre = incl - tot;
  if (4 * lane < k.Q) {
    *reinterpret_cast<float4*>(k.dtq + row + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(k.dacs + row + 4 * lane) =
        make_float4(pre + a[0], pre + a[1], pre + a[2], pre + a[3]);
  }
}

// ---- 2. chunk states -----------------------------------------------------------------

// MODE 0 (forward): st_c = sum_l x_l (dt'_l e^{S_last - S_l} [seq_l == seq_last]) B_l^T.
// MODE 1 (backward): dhl_c = sum_l dy_l (e^{S_l} [seq_l == seq before the chunk]) C_l^T,
// the gradient of the state entering chunk c from the chunk's own outputs.
// MODE 2 (varlen states, batch 1; chunk_state_varlen, ssd_chunk_state.py:589-660): for the
// sequence [start, end) and c the chunk of step end - 1, with e = end - 1 - c Q,
// state = sum_{l in c, l >= start} x_l (dt'_l e^{S_e - S_l}) B_l^T (+ e^{S_e} H_c when the
// sequence began before chunk c), written in the input type.
//
// Software pipeline over 32-step slices: the global loads of slice i + 1 (x rows, B rows and
// their weights) go to registers while the MFMAs of slice i run; the registers are written,
// transposed and weighted, to the other half of a double LDS buffer, one barrier per slice.
// (With a single buffer, when two would not fit in 64 KB, a second barrier guards it.)
// Occupancy target of 4 waves per SIMD for headdim 64 x dstate 128 (Mamba-2's default),
// which the compiler otherwise lays out at 140-144 registers (3 waves; the 4-wave layout
// measured 172 -> 141 us), and for the small tiles it changes nothing for.  Larger tiles keep
// the default: at 128 registers they would spill.
template <typename T, int P, int N, int MODE>
__global__ void __launch_bounds__(kThreads)
    __attribute__((amdgpu_waves_per_eu((P * N <= 4096 || (P == 64 && N == 128)) ? 4 : 1)))
    ssd_chunk_state(SsdK k) {
  typedef Mma<T> M;
  typedef typename M::Raw Raw;
  constexpr int VE = M::kVe;
  constexpr int NTN = N / 16;
  constexpr int NT = (P / 16) * NTN;
  constexpr int TPW = (NT + 3) / 4;
  constexpr int ES = sizeof(Raw);
  // 16-bit types: slices stay row-major in LDS (16-byte stores, rows l) and the MFMA operands
  // come through transposing reads; fp32: slices are written transposed (rows p / n).
  constexpr bool TR = ES == 2;
  constexpr int XPT = P + 16, BPT = N + 16;                      // row-major pitches (TR)
  constexpr int SLICE_BYTES = TR ? kKs * (XPT + BPT) * ES : (P + N) * kLp * ES;
  constexpr int NB = 2 * SLICE_BYTES <= 65536 ? 2 : 1;
  constexpr int XC = kKs * (P / VE), BC = kKs * (N / VE);       // 16-byte chunks per slice
  constexpr int XL = (XC + kThreads - 1) / kThreads, BL = (BC + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) char smem[NB * SLICE_BYTES];
  Raw (*xs)[P][kLp] = reinterpret_cast<Raw (*)[P][kLp]>(smem);
  Raw (*bs)[N][kLp] = reinterpret_cast<Raw (*)[N][kLp]>(smem + NB * P * kLp * ES);
  Raw (*xr)[kKs][XPT] = reinterpret_cast<Raw (*)[kKs][XPT]>(smem);
  Raw (*br)[kKs][BPT] = reinterpret_cast<Raw (*)[kKs][BPT]>(smem + NB * kKs * XPT * ES);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // work id -> (head fastest, chunk, batch): the heads of one chunk share its B (C) rows;
  // MODE 2: (head fastest, sequence)
  const int64_t wid = xcd_work_id();
  const int64_t hh = wid % k.H;
  int64_t c, b;
  int lim, rstart = 0;        // rows [rstart, lim) of the chunk contribute
  bool carry = false;         // MODE 2: add the decayed entering state
  if constexpr (MODE == 2) {
    const int64_t si = wid / k.H;
    const int64_t s0 = k.cu[si], s1 = k.cu[si + 1];
    const bool ok = 0 <= s0 && s0 < s1 && s1 <= k.L;
    b = 0;
    c = ok ? (s1 - 1) / k.Q : 0;
    lim = ok ? (int)(s1 - c * k.Q) : 0;
    rstart = ok ? (int)max(s0 - c * k.Q, (int64_t)0) : 0;
    carry = ok && s0 < c * k.Q;
  } else {
    c = (wid / k.H) % k.K;
    b = wid / (k.H * k.K);
    lim = (int)min(k.Q, k.L - c * k.Q);
  }
  const int64_t g = hh / k.hpg;
  const int64_t t0 = c * k.Q;
  const float* sq = k.dacs + ((b * k.H + hh) * k.K + c) * k.Q;
  const float* dq = k.dtq + ((b * k.H + hh) * k.K + c) * k.Q;
  const float s_last = MODE == 2 ? (lim > 0 ? sq[lim - 1] : 0.f) : sq[k.Q - 1];
  const int32_t seq_ref = (!k.has_seq || MODE == 2) ? 0
                          : MODE == 0 ? seq_at(k, b, t0 + lim - 1)
                                      : (c > 0 ? seq_at(k, b, t0 - 1) : 0);
  const int64_t* sxr = MODE != 1 ? k.sx : k.sdy;
  const int64_t* sbr = MODE != 1 ? k.sB : k.sC;
  const char* xbase = (const char*)(MODE != 1 ? k.x : k.dy) + (b * sxr[0] + t0 * sxr[1] + hh * sxr[2]) * ES;
  const char* bbase = (const char*)(MODE != 1 ? k.Bm : k.Cm) + (b * sbr[0] + t0 * sbr[1] + g * sbr[2]) * ES;

  Raw xv[XL][VE], bv[BL][VE];
  // The weight inputs of each B row (dt', the cumsum, the seq_idx value) stay raw until the
  // slice is written to LDS: a weight formed right after its loads would wait for them there,
  // one full memory latency per slice.
  float dqv[BL], sqv[BL];
  int32_t sqi[BL];
  // Loads of the slice starting at l0 into registers; rows past the sequence end read as 0.
  auto fetch = [&](int l0) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      const int r = e / (P / VE), col = (e % (P / VE)) * VE;
      if (e < XC && l0 + r < lim) load16<T>(xbase + ((l0 + r) * sxr[1] + col) * ES, xv[i]);
      else
#pragma unroll
        for (int q = 0; q < VE; ++q) xv[i][q] = M::to_raw(0.f);
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) {
      const int e = tid + i * kThreads;
      const int r = e / (N / VE), col = (e % (N / VE)) * VE;
      const int l = l0 + r;
      dqv[i] = 0.f;  // weight 0 past the sequence end
      sqv[i] = 0.f;
      sqi[i] = seq_ref;
      if (e < BC && l < lim) {
        load16<T>(bbase + (l * sbr[1] + col) * ES, bv[i]);
        dqv[i] = MODE != 1 ? dq[l] : 1.f;
        sqv[i] = sq[l];
        if (MODE != 2 && k.has_seq) sqi[i] = seq_at(k, b, t0 + l);
        if (MODE == 2 && l < rstart) dqv[i] = 0.f;
      } else {
#pragma unroll
        for (int q = 0; q < VE; ++q) bv[i][q] = M::to_raw(0.f);
      }
    }
  };

  f4 acc[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

  const int nsl = (lim + kKs - 1) / kKs;
  fetch(0);
  for (int sl = 0; sl < nsl; ++sl) {
    const int buf = NB == 2 ? (sl & 1) : 0;
    if (NB == 1 && sl > 0) __syncthreads();  // the single buffer is consumed
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      if (e < XC) {
        const int r = e / (P / VE), col = (e % (P / VE)) * VE;
        if constexpr (TR) {
          *reinterpret_cast<u4*>(&xr[buf][r][col]) = *reinterpret_cast<const u4*>(xv[i]);
        } else {
#pragma unroll
          for (int q = 0; q < VE; ++q) xs[buf][col + q][r] = xv[i][q];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) {
      const int e = tid + i * kThreads;
      if (e < BC) {
        const int r = e / (N / VE), col = (e % (N / VE)) * VE;
        float wgt = dqv[i] * exp_split(MODE != 1 ? s_last - sqv[i] : sqv[i]);
        if (MODE != 2 && k.has_seq && sqi[i] != seq_ref) wgt = 0.f;
        Raw o[VE];
#pragma unroll
        for (int q = 0; q < VE; ++q) o[q] = M::to_raw(M::from_raw(bv[i][q]) * wgt);
        if constexpr (TR) {
          *reinterpret_cast<u4*>(&br[buf][r][col]) = *reinterpret_cast<const u4*>(o);
        } else {
#pragma unroll
          for (int q = 0; q < VE; ++q) bs[buf][col + q][r] = o[q];
        }
      }
    }
    __syncthreads();
    if (sl + 1 < nsl) fetch((sl + 1) * kKs);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int ti = w + 4 * i;
      if (ti < NT) {
        const int pt = ti / NTN, nt = ti % NTN;
        typename M::Frag a, bf;
        if constexpr (TR) {
          a = M::load_tr(&xr[buf][0][pt * 16], XPT, lane);
          bf = M::load_tr(&br[buf][0][nt * 16], BPT, lane);
        } else {
          a = M::load_row(&xs[buf][pt * 16 + (lane & 15)][0], lane);
          bf = M::load_row(&bs[buf][nt * 16 + (lane & 15)][0], lane);
        }
        M::mma(acc[i], a, bf);
      }
    }
  }
  if constexpr (MODE == 2) {
    const Raw* hin = (const Raw*)k.hs + ((b * k.K + c) * k.H + hh) * (int64_t)(P * N);
    const float sc = carry ? exp_split(s_last) : 0.f;
    Raw* out = (Raw*)k.vst + ((wid / k.H) * k.H + hh) * (k.Pa * k.Na);  // [nseq, H, Pa, Na]
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int ti = w + 4 * i;
      if (ti < NT) {
        const int pt = ti / NTN, nt = ti % NTN;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int pr = pt * 16 + 4 * (lane >> 4) + j, nc = nt * 16 + (lane & 15);
          const float v = carry ? fmaf(M::from_raw(hin[pr * N + nc]), sc, acc[i][j]) : acc[i][j];
          if (pr < k.Pa && nc < k.Na) out[pr * k.Na + nc] = M::to_raw(v);
        }
      }
    }
  } else {
    float* out = (MODE == 0 ? k.st : k.dhl) + ((b * k.K + c) * k.H + hh) * (int64_t)(P * N);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int ti = w + 4 * i;
      if (ti < NT) {
        const int pt = ti / NTN, nt = ti % NTN;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          out[(pt * 16 + 4 * (lane >> 4) + j) * N + nt * 16 + (lane & 15)] = acc[i][j];
      }
    }
  }
}

// ---- 3. state passing across chunks --------------------------------------------------

// Sequential over chunks, 4 state elements per thread; each chunk's inputs (the chunk
// state and its decay) are loaded two chunks ahead, so the chain's loads overlap.
constexpr int kSpEpt = 4;  // elements per thread (P N is a multiple of 1024)

template <typename T>
__global__ void __launch_bounds__(kThreads) ssd_state_pass(SsdK k) {
  typedef typename Mma<T>::Raw Raw;
  const int64_t PN = k.P * k.N;
  const int64_t hh = blockIdx.y, b = blockIdx.z;
  int64_t e[kSpEpt];
  float H[kSpEpt];
#pragma unroll
  for (int i = 0; i < kSpEpt; ++i) {
    e[i] = (int64_t)blockIdx.x * (kThreads * kSpEpt) + threadIdx.x + i * kThreads;
    const int64_t p = e[i] / k.N, n = e[i] % k.N;
    H[i] = (k.has_init && p < k.Pa && n < k.Na)
               ? k.init[b * k.sinit[0] + hh * k.sinit[1] + p * k.sinit[2] + n * k.sinit[3]] : 0.f;
  }
  Raw* hs = (Raw*)k.hs;
  const float* sl = k.dacs + (b * k.H + hh) * k.K * k.Q + k.Q - 1;  // S_last of chunk c: sl[c * Q]
  auto ofs = [&](int64_t c) { return ((b * k.K + c) * k.H + hh) * PN; };
  float sa[kSpEpt], sb[kSpEpt], la = 0.f, lb = 0.f;
  auto fetch = [&](int64_t c, float (&v)[kSpEpt], float& l) {
    if (c >= k.K) return;
#pragma unroll
    for (int i = 0; i < kSpEpt; ++i) v[i] = k.st[ofs(c) + e[i]];
    l = sl[c * k.Q];
  };
  fetch(0, sa, la);
  fetch(1, sb, lb);
  int32_t seq_prev = 0;
  auto step = [&](int64_t c, float (&v)[kSpEpt], float& l) {
    float scale = exp_split(l);
    if (k.has_seq) {
      const int32_t sn = seq_at(k, b, min((c + 1) * k.Q, k.L) - 1);
      if (sn != seq_prev) scale = 0.f;
      seq_prev = sn;
    }
    const int64_t o = ofs(c);
    float cur[kSpEpt];
#pragma unroll
    for (int i = 0; i < kSpEpt; ++i) cur[i] = v[i];
    fetch(c + 2, v, l);
#pragma unroll
    for (int i = 0; i < kSpEpt; ++i) {
      hs[o + e[i]] = Mma<T>::to_raw(H[i]);
      H[i] = fmaf(scale, H[i], cur[i]);
    }
  };
  for (int64_t c = 0; c < k.K; c += 2) {
    step(c, sa, la);
    if (c + 1 < k.K) step(c + 1, sb, lb);
  }
  if (k.final_states) {  // [Bsz, H, Pa, Na]
#pragma unroll
    for (int i = 0; i < kSpEpt; ++i) {
      const int64_t p = e[i] / k.N, n = e[i] % k.N;
      if (p < k.Pa && n < k.Na) k.final_states[((b * k.H + hh) * k.Pa + p) * k.Na + n] = H[i];
    }
  }
}

// ---- 4. C B^T within each chunk ------------------------------------------------------

template <typename T, int N>
__global__ void __launch_bounds__(kThreads) ssd_bmm(SsdK k) {
  typedef Mma<T> M;
  typedef typename M::Raw Raw;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int ti = 0, rem = (int)blockIdx.x;  // lower-triangle 64x64 tile (ti, tj), tj <= ti
  while (rem > ti) { rem -= ti + 1; ++ti; }
  const int tj = rem;
  const int64_t c = blockIdx.y, b = blockIdx.z / k.G, g = blockIdx.z % k.G;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  const Raw* Cb = (const Raw*)k.Cm + b * k.sC[0] + t0 * k.sC[1] + g * k.sC[2];
  const Raw* Bb = (const Raw*)k.Bm + b * k.sB[0] + t0 * k.sB[1] + g * k.sB[2];
  const int row = ti * 64 + 16 * w + (lane & 15);
  f4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int n0 = 0; n0 < N; n0 += kKs) {
    // rows / columns past lim read the last valid row; their CB entries are zeroed below
    const typename M::Frag a = M::load_row(Cb + min(row, lim - 1) * k.sC[1] + n0, lane);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int s = tj * 64 + 16 * ct + (lane & 15);
      const typename M::Frag bf = M::load_row(Bb + min(s, lim - 1) * k.sB[1] + n0, lane);
      M::mma(acc[ct], a, bf);
    }
  }
  float* out = k.cb + ((b * k.K + c) * k.G + g) * k.Q * k.Q;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = ti * 64 + 16 * w + 4 * (lane >> 4) + j;
      const int s = tj * 64 + 16 * ct + (lane & 15);
      float v = acc[ct][j];
      if (!(l < lim && s < lim)) v = 0.f;
      else if (k.has_seq && seq_at(k, b, t0 + l) != seq_at(k, b, t0 + s)) v = 0.f;
      out[(int64_t)l * k.Q + s] = v;
    }
  }
}

// ---- 5. chunk scan -------------------------------------------------------------------

// Block: 64 rows (steps) of one chunk and head, 4 waves of 16 rows, all of headdim.
// The intra-chunk product runs as a software pipeline over stages of SUB MFMA K steps: the
// x rows and the wave's CB values of stage i + 1 are loaded to registers while stage i's
// MFMAs run, x goes transposed to the other half of a double LDS buffer, one barrier per
// stage.  The decay e^{S_l - S_s} is exp2((S_l - S_s) log2 e), as the reference's tl.exp:
// the difference is taken first, since the cumsums themselves can reach thousands and
// scaling them before subtracting would add their rounding to the exponent.  y is staged
// through LDS (reusing the x buffer) so that the D skip, the z gate and the stores run on
// 16-byte rows.
template <typename T, int P, int N>
__global__ void __launch_bounds__(kThreads) ssd_chunk_scan(SsdK k) {
  typedef Mma<T> M;
  typedef typename M::Raw Raw;
  constexpr int VE = M::kVe;
  constexpr int PT = P / 16;
  constexpr int ES = sizeof(Raw);
  constexpr int SUB = (ES == 2 || P <= 64) ? 2 : 1;       // MFMA K steps per stage
  constexpr int KST = SUB * kKs;                           // steps per stage
  constexpr int LP = KST + 8;                              // LDS row pitch, 16-byte rows
  constexpr int XC = KST * (P / VE);                       // 16-byte x chunks per stage
  constexpr int XL = (XC + kThreads - 1) / kThreads;
  constexpr int YP = P + 4;                                // y staging pitch (floats)
  constexpr int HCH = N < 128 ? N : ((ES == 4 && P == 128) ? 64 : 128);  // H columns per stage
  constexpr int HP = HCH + 8;                              // H staging pitch, 16-byte rows
  constexpr bool TR = ES == 2;                             // row-major x + transposing reads
  constexpr int XPT = P + 16;                              // row-major x pitch (TR)
  constexpr int XS_BYTES = TR ? 2 * KST * XPT * ES : 2 * P * LP * ES;
  constexpr int YS_BYTES = 64 * YP * 4, HS_BYTES = P * HP * ES;
  // 16-bit types with 64-step stages (headdim <= 64): the intra loop's last stage is the
  // block's own 64 rows of x, so the D skip reads them from that LDS buffer instead of global
  // memory, and y gets its own staging area after the x buffers.
  constexpr bool XKEEP = TR && KST == 64 && P <= 64;
  constexpr int SM_A = XKEEP ? XS_BYTES + YS_BYTES : (XS_BYTES > YS_BYTES ? XS_BYTES : YS_BYTES);
  constexpr int SM_BYTES = SM_A > HS_BYTES ? SM_A : HS_BYTES;
  __shared__ __attribute__((aligned(16))) char smem[SM_BYTES];
  __shared__ float sls[2][KST], dls[2][KST];
  Raw (*xs)[P][LP] = reinterpret_cast<Raw (*)[P][LP]>(smem);
  Raw (*xr)[KST][XPT] = reinterpret_cast<Raw (*)[KST][XPT]>(smem);
  float (*ys)[YP] = reinterpret_cast<float (*)[YP]>(smem + (XKEEP ? XS_BYTES : 0));
  Raw (*hsm)[HP] = reinterpret_cast<Raw (*)[HP]>(smem);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // work id -> (head fastest, row tile, chunk, batch): one (batch, chunk)'s blocks, which
  // share its CB tile, and one head's row tiles, which share its passed state, run together
  const int64_t wid = xcd_work_id();
  const int64_t hh = wid % k.H;
  const int lt = (int)((wid / k.H) % (k.Q / 64));
  const int64_t c = (wid / (k.H * (k.Q / 64))) % k.K, b = wid / (k.H * (k.Q / 64) * k.K);
  const int64_t g = hh / k.hpg;
  const int64_t t0 = c * k.Q;
  const int lim = (int)min(k.Q, k.L - t0);
  if (lt * 64 >= lim) return;  // whole block
  const float* sq = k.dacs + ((b * k.H + hh) * k.K + c) * k.Q;
  const float* dq = k.dtq + ((b * k.H + hh) * k.K + c) * k.Q;
  const int rowbase = lt * 64 + 16 * w;
  const int row = rowbase + (lane & 15);  // A-operand row of this lane
  const float* cbrow = k.cb + ((b * k.K + c) * k.G + g) * k.Q * k.Q + (int64_t)row * k.Q;
  const char* xbase = (const char*)k.x + (b * k.sx[0] + t0 * k.sx[1] + hh * k.sx[2]) * ES;
  const int s_end = min(lt * 64 + 64, lim);
  const int nst = (s_end + KST - 1) / KST;

  Raw xv[XL][VE];
  float cbv[SUB][8];
  float sv = 0.f, dv = 0.f;
  auto fetch = [&](int s0) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      const int r = e / (P / VE), col = (e % (P / VE)) * VE;
      if (e < XC && s0 + r < lim) load16<T>(xbase + ((s0 + r) * k.sx[1] + col) * ES, xv[i]);
      else
#pragma unroll
        for (int q = 0; q < VE; ++q) xv[i][q] = M::to_raw(0.f);
    }
    if (tid < KST) {  // rows of the chunk past lim hold S and dt' of 0 / the last step
      sv = sq[s0 + tid];
      dv = dq[s0 + tid];
    }
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks) {
      if constexpr (TR) {
        // this lane's 8 consecutive CB values of the slice, as two 16-byte loads: 16-byte
        // aligned (the chunk size is a multiple of 64) and inside the chunk's Q x Q tile
        // (s0 + KST <= Q); slices past the wave's rows are loaded but not used
        const float4* src = reinterpret_cast<const float4*>(cbrow + s0 + ks * kKs + 8 * (lane >> 4));
        const float4 lo = src[0], hi = src[1];
        cbv[ks][0] = lo.x; cbv[ks][1] = lo.y; cbv[ks][2] = lo.z; cbv[ks][3] = lo.w;
        cbv[ks][4] = hi.x; cbv[ks][5] = hi.y; cbv[ks][6] = hi.z; cbv[ks][7] = hi.w;
      } else {
        const bool reach = s0 + ks * kKs <= rowbase + 15;  // wave-uniform
#pragma unroll
        for (int j = 0; j < 8; ++j) cbv[ks][j] = reach ? cbrow[s0 + ks * kKs + M::kidx(lane, j)] : 0.f;
      }
    }
  };
  fetch(0);
  // Values used only after the state term: loaded here, with the first stage, so that no
  // later step waits a full memory latency for them.
  // Rows < Q are in bounds; rows past lim are masked where these are used.  Loaded without a
  // condition: a conditional load would wait for itself under its branch.
  const float s_row = sq[row];  // S of this lane's A-operand row
  float s_acc[4];               // S of this lane's accumulator rows
#pragma unroll
  for (int j = 0; j < 4; ++j) s_acc[j] = sq[rowbase + 4 * (lane >> 4) + j];
  const float D_head = (k.has_D && !k.D_hdim) ? k.Dp[hh * k.sD[0]] : 0.f;

  f4 acc[PT];
#pragma unroll
  for (int i = 0; i < PT; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

  // (a) contribution of the state entering the chunk: e^{S_l} C_l H_c^T.  H (shared by the
  // block's 4 waves) is staged through LDS in column stages of HCH with coalesced 16-byte
  // loads; each wave's C fragments come straight from global memory.  The condition is
  // block-uniform, so the barriers inside are too.
  if (c > 0 || k.has_init) {
    // rows past lim read the last valid row: their outputs are scaled by f = 0 below
    const Raw* Crow = (const Raw*)k.Cm + b * k.sC[0] + (t0 + min(row, lim - 1)) * k.sC[1] + g * k.sC[2];
    const Raw* H = (const Raw*)k.hs + ((b * k.K + c) * k.H + hh) * (int64_t)(P * N);
    constexpr int HC = P * (HCH / VE);
    constexpr int HL = (HC + kThreads - 1) / kThreads;
#pragma unroll
    for (int nc = 0; nc < N; nc += HCH) {
      typename M::Frag af[HCH / kKs];
#pragma unroll
      for (int i = 0; i < HCH / kKs; ++i) af[i] = M::load_row(Crow + nc + i * kKs, lane);
      u4 hv[HL];
#pragma unroll
      for (int i = 0; i < HL; ++i) {
        const int e = tid + i * kThreads;
        const int p = e / (HCH / VE), col = (e % (HCH / VE)) * VE;
        if (e < HC) hv[i] = *reinterpret_cast<const u4*>(H + p * N + nc + col);
      }
      if (nc > 0) __syncthreads();  // the previous stage is consumed
#pragma unroll
      for (int i = 0; i < HL; ++i) {
        const int e = tid + i * kThreads;
        const int p = e / (HCH / VE), col = (e % (HCH / VE)) * VE;
        if (e < HC) *reinterpret_cast<u4*>(&hsm[p][col]) = hv[i];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < HCH / kKs; ++i)
#pragma unroll
        for (int pt = 0; pt < PT; ++pt)
          M::mma(acc[pt], af[i], M::load_row(&hsm[pt * 16 + (lane & 15)][i * kKs], lane));
    }
    __syncthreads();  // H consumed before the intra loop writes x over it
    const int32_t seq_prev = (k.has_seq && c > 0) ? seq_at(k, b, t0 - 1) : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int l = rowbase + 4 * (lane >> 4) + j;
      float f = 0.f;
      if (l < lim) {
        f = exp_split(s_acc[j]);
        if (k.has_seq && seq_at(k, b, t0 + l) != seq_prev) f = 0.f;
      }
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) acc[pt][j] *= f;
    }
  }

  // (b) within the chunk: sum_{s <= l} CB[l, s] e^{S_l - S_s} dt'_s x_s
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    const int s0 = st * KST;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kThreads;
      if (e < XC) {
        const int r = e / (P / VE), col = (e % (P / VE)) * VE;
        if constexpr (TR) {
          *reinterpret_cast<u4*>(&xr[buf][r][col]) = *reinterpret_cast<const u4*>(xv[i]);
        } else {
#pragma unroll
          for (int q = 0; q < VE; ++q) xs[buf][col + q][r] = xv[i][q];
        }
      }
    }
    if (tid < KST) {
      sls[buf][tid] = sv;
      dls[buf][tid] = dv;
    }
    float cbc[SUB][8];
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) cbc[ks][j] = cbv[ks][j];
    __syncthreads();
    if (st + 1 < nst) fetch(s0 + KST);
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks) {
      if (s0 + ks * kKs <= rowbase + 15) {  // wave-uniform: the slice reaches this wave's rows
        float m[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int si = ks * kKs + M::kidx(lane, j);
          const int s = s0 + si;
          const bool on = s <= row && row < lim && s < lim;
          const float v = cbc[ks][j] * fast_exp2((s_row - sls[buf][si]) * kLog2e) * dls[buf][si];
          m[j] = on ? v : 0.f;
        }
        const typename M::Frag a = M::from_float(m);
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
          if constexpr (TR) M::mma(acc[pt], a, M::load_tr(&xr[buf][ks * kKs][pt * 16], XPT, lane));
          else M::mma(acc[pt], a, M::load_row(&xs[buf][pt * 16 + (lane & 15)][ks * kKs], lane));
        }
      }
    }
  }

  // (c) y through LDS, then the D skip, z gate and 16-byte stores
  __syncthreads();  // every wave is done reading x from the buffer ys reuses
#pragma unroll
  for (int pt = 0; pt < PT; ++pt)
#pragma unroll
    for (int j = 0; j < 4; ++j) ys[16 * w + 4 * (lane >> 4) + j][pt * 16 + (lane & 15)] = acc[pt][j];
  __syncthreads();
  constexpr int YC = 64 * (P / VE);
  for (int e = tid; e < YC; e += kThreads) {
    const int r = e / (P / VE), col = (e % (P / VE)) * VE;
    const int l = lt * 64 + r;
    if (l >= lim) continue;
    const int64_t t = t0 + l;
    float y[VE];
#pragma unroll
    for (int q = 0; q < VE; ++q) y[q] = ys[r][col + q];
    if (k.has_D) {
      Raw xl[VE];
      if constexpr (XKEEP)  // the last stage (rows lt * 64 ..) is still in its LDS buffer
        *reinterpret_cast<u4*>(xl) = *reinterpret_cast<const u4*>(&xr[(nst - 1) & 1][r][col]);
      else
        load16<T>(xbase + (l * k.sx[1] + col) * ES, xl);
#pragma unroll
      for (int q = 0; q < VE; ++q) {
        const float Dv = !k.D_hdim ? D_head
                         : col + q < k.Pa ? k.Dp[hh * k.sD[0] + (col + q) * k.sD[1]] : 0.f;
        y[q] = fmaf(Dv, M::from_raw(xl[q]), y[q]);
      }
    }
    Raw o[VE];
    if (k.has_z) {
      Raw zr[VE];
      load16<T>((const char*)k.z + (b * k.sz[0] + t * k.sz[1] + hh * k.sz[2] + col) * ES, zr);
      if (k.out_x) {
#pragma unroll
        for (int q = 0; q < VE; ++q) o[q] = M::to_raw(y[q]);
        *reinterpret_cast<uint4*>((char*)k.out_x + (b * k.soutx[0] + t * k.soutx[1] + hh * k.soutx[2] + col) * ES) =
            *reinterpret_cast<const uint4*>(o);
      }
#pragma unroll
      for (int q = 0; q < VE; ++q) {
        const float zz = M::from_raw(zr[q]);
        y[q] *= zz * sigmoidf_(zz);
      }
    }
#pragma unroll
    for (int q = 0; q < VE; ++q) o[q] = M::to_raw(y[q]);
    *reinterpret_cast<uint4*>((char*)k.out + (b * k.sout[0] + t * k.sout[1] + hh * k.sout[2] + col) * ES) =
        *reinterpret_cast<const uint4*>(o);
  }
}

// ---- dispatch ------------------------------------------------------------------------

template <typename T, int P, int N>
hipError_t ssd_prep_pn(const SsdK& k, hipStream_t st) {
  hipError_t e;
  hipLaunchKernelGGL((ssd_cumsum), dim3((unsigned)k.K, (unsigned)k.H, (unsigned)k.Bsz), dim3(kWave),
                     0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_chunk_state<T, P, N, 0>), dim3((unsigned)(k.K * k.H * k.Bsz)),
                     dim3(kThreads), 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_state_pass<T>), dim3((unsigned)(P * N / (kThreads * kSpEpt)),
                     (unsigned)k.H, (unsigned)k.Bsz), dim3(kThreads), 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int qt = (int)(k.Q / 64);
  hipLaunchKernelGGL((ssd_bmm<T, N>), dim3((unsigned)(qt * (qt + 1) / 2), (unsigned)k.K,
                     (unsigned)(k.Bsz * k.G)), dim3(kThreads), 0, st, k);
  return hipGetLastError();
}

template <typename T, int P, int N>
hipError_t ssd_scan_pn(const SsdK& k, hipStream_t st) {
  const int qt = (int)(k.Q / 64);
  hipLaunchKernelGGL((ssd_chunk_scan<T, P, N>), dim3((unsigned)(qt * k.K * k.Bsz * k.H)), dim3(kThreads),
                     0, st, k);
  return hipGetLastError();
}

template <typename T, int P, int N>
hipError_t ssd_varlen_pn(const SsdK& k, hipStream_t st) {
  hipLaunchKernelGGL((ssd_chunk_state<T, P, N, 2>), dim3((unsigned)(k.nseq * k.H)), dim3(kThreads), 0, st, k);
  return hipGetLastError();
}

template <typename T, int P, int N>
hipError_t ssd_dstates_pn(const SsdK& k, hipStream_t st) {
  hipLaunchKernelGGL((ssd_chunk_state<T, P, N, 1>), dim3((unsigned)(k.K * k.H * k.Bsz)),
                     dim3(kThreads), 0, st, k);
  return hipGetLastError();
}

// Calls F<T, P, N>::run(k, st) for the problem's dtype, headdim and dstate.
#define S6_SSD_DISPATCH(FN)                                                               \
  template <typename T, int P>                                                            \
  hipError_t FN##_p(const SsdK& k, hipStream_t st) {                                      \
    switch (k.N) {                                                                        \
      case 32: return FN##_pn<T, P, 32>(k, st);                                           \
      case 64: return FN##_pn<T, P, 64>(k, st);                                           \
      case 128: return FN##_pn<T, P, 128>(k, st);                                         \
      case 256: return FN##_pn<T, P, 256>(k, st);                                         \
      default: return hipErrorInvalidValue;                                               \
    }                                                                                     \
  }                                                                                       \
  template <typename T>                                                                   \
  hipError_t FN##_t(const SsdK& k, hipStream_t st) {                                      \
    switch (k.P) {                                                                        \
      case 32: return FN##_p<T, 32>(k, st);                                               \
      case 64: return FN##_p<T, 64>(k, st);                                               \
      case 128: return FN##_p<T, 128>(k, st);                                             \
      default: return hipErrorInvalidValue;                                               \
    }                                                                                     \
  }                                                                                       \
  hipError_t FN(const SsdK& k, hipStream_t st) {                                          \
    if (k.io == S6_BF16) return FN##_t<bf16>(k, st);                                      \
    if (k.io == S6_F16) return FN##_t<f16>(k, st);                                        \
    if (k.io == S6_F32) return FN##_t<float>(k, st);                                      \
    return hipErrorInvalidValue;                                                          \
  }

S6_SSD_DISPATCH(ssd_prep)
S6_SSD_DISPATCH(ssd_scan)
S6_SSD_DISPATCH(ssd_dstates)
S6_SSD_DISPATCH(ssd_varlen)

}  // namespace

hipError_t launch_ssd_prep(const SsdK& k, hipStream_t st) { return ssd_prep(k, st); }

hipError_t launch_ssd_dstates(const SsdK& k, hipStream_t st) { return ssd_dstates(k, st); }

hipError_t launch_ssd_fwd(const SsdK& k, hipStream_t st, void* const* ev) {
  hipError_t e = ssd_prep(k, st);
  if (e != hipSuccess || (e = record_event(ev, 0, st)) != hipSuccess) return e;
  if ((e = ssd_scan(k, st)) != hipSuccess) return e;
  if ((e = record_event(ev, 1, st)) != hipSuccess) return e;
  return k.vst != nullptr ? ssd_varlen(k, st) : hipSuccess;
}

}  // namespace s6
