// Internal launch interface between the C ABI (s6_abi.cpp) and the HIP kernels, and the
// device helpers the kernel files share.
#pragma once
#include "s6_common.h"
#include "causal_conv1d.h"

namespace s6 {

// Sequence bookkeeping for packed varlen input: index into cu_seqlens of the first
// sequence start >= t0, and that start (INT64_MAX past the last one).
struct SeqCursor {
  int32_t idx;
  int64_t pending;
};

__device__ inline SeqCursor seq_cursor_at(const int32_t* cu, int32_t nseq, int64_t t0) {
  int32_t lo = 0, hi = nseq + 1;  // first i with cu[i] >= t0 (cu non-decreasing)
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if ((int64_t)cu[mid] < t0) lo = mid + 1; else hi = mid;
  }
  SeqCursor s;
  s.idx = lo;
  s.pending = (lo <= nseq) ? (int64_t)cu[lo] : INT64_MAX;
  return s;
}

// True when a sequence starts at some step of [t0, t1).
__device__ inline bool range_has_start(const int32_t* cu, int32_t nseq, int64_t t0, int64_t t1) {
  return seq_cursor_at(cu, nseq, t0).pending < t1;
}

// Bit i set when a sequence starts at step ts + i, for i in [0, te - ts), te - ts <= 32.
// Offsets outside [ts, te) set no bit, so a vector that is not non-decreasing (which the
// host rejects before launching) cannot produce an out-of-range shift.
__device__ inline uint32_t start_mask(const int32_t* cu, int32_t nseq, int64_t ts, int64_t te) {
  SeqCursor s = seq_cursor_at(cu, nseq, ts);
  uint32_t m = 0;
  for (int32_t i = s.idx; i <= nseq && (int64_t)cu[i] < te; ++i) {
    const int64_t off = (int64_t)cu[i] - ts;
    if (off >= 0 && off < 32) m |= 1u << (uint32_t)off;
  }
  return m;
}

// Reverse cursor for kernels that visit [t0, t1) in consecutive decreasing ranges: pend is the
// largest sequence start below the ranges still to visit (-1 when there is none), hi - 1 its
// index in cu_seqlens.  start_mask_rev then costs one compare per range and one load per
// start passed, where start_mask searches cu_seqlens again for every range.
struct SeqCursorRev {
  int32_t hi;
  int64_t pend;
};

__device__ inline SeqCursorRev seq_cursor_rev_at(const int32_t* cu, int32_t nseq, int64_t t1) {
  const SeqCursor s = seq_cursor_at(cu, nseq, t1);  // first i with cu[i] >= t1
  SeqCursorRev r;
  r.hi = s.idx;
  r.pend = s.idx > 0 ? (int64_t)cu[s.idx - 1] : -1;
  return r;
}

// The bits start_mask(cu, nseq, ts, te) sets, for te = the previous call's ts (the first call:
// seq_cursor_rev_at's t1); offsets past 31 set no bit.  Every iteration lowers hi, so the loop
// ends for any vector.
__device__ inline uint32_t start_mask_rev(SeqCursorRev& r, const int32_t* cu, int64_t ts) {
  uint32_t m = 0;
  while (r.hi > 0 && r.pend >= ts) {
    const int64_t off = r.pend - ts;
    if (off < 32) m |= 1u << (uint32_t)off;
    --r.hi;
    r.pend = r.hi > 0 ? (int64_t)cu[r.hi - 1] : -1;
  }
  return m;
}

// Stores the first N (<= NS) states of one lane to a contiguous fp32 row.
template <int NS>
__device__ inline void store_state(float* dst, const float (&h)[NS], int N) {
  if (N == NS && (NS % 4) == 0) {
#pragma unroll
    for (int n = 0; n < NS; n += 4)
      *reinterpret_cast<float4*>(dst + n) = make_float4(h[n], h[n + 1], h[n + 2], h[n + 3]);
  } else {
    // Unrolled over NS with a predicate: a runtime-bounded loop would index h dynamically
    // and force the whole state array out of registers into scratch.
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) dst[n] = h[n];
  }
}

// Parameter block of the backward kernels (strides in elements).
struct BwdK {
  int64_t Bsz, D, L, N, G;
  int64_t su[3], sdl[3], sz[3], sdo[3], sout[3], sdu[3], sddl[3], sdz[3];
  int64_t sA[2], sD, sbias;
  int64_t sB[4], sC[4];
  int64_t sdB[4], sdC[4];
  const void* u; const void* delta; const void* z; const void* dout; const void* out;
  const float* A; const float* Dp; const float* bias;
  const void* Bm; const void* Cm;
  const int32_t* cu; int32_t nseq;
  const float* x_ckpt; int64_t nck;   // [Bsz, nck, D, N], as written by the forward
  int64_t sck[3];                     // its batch, checkpoint and dim strides
  void* du; void* ddelta; void* dz;
  void* out_z; int64_t soz[3];   // out * silu(z) (recompute_out_z), NULL: not written
  float* dA; float* dD; float* dbias; float* dB; float* dC;
  int64_t sdA[2], sdD, sdbias;
  float* ws_g;   // [Bsz*D, K, N]     reverse chunk summaries, then carried-in gradients
  float* ws_s;   // [Bsz*D, K]        sum of Delta over each chunk
  int32_t* ws_r; // [Bsz*D, K]        1 if a sequence starts inside the chunk (varlen only)
  float* ws_pB;  // [Bsz, G, nJ, L, NPr]  per-64-channel-block partial dB
  float* ws_pC;  // [Bsz, G, nJ, L, NPr]  per-64-channel-block partial dC
  float* ws_s1;  // unused (kept so that the kernel-argument layout, and with it the
  float* ws_s2;  // register allocation of the hot kernels, stays as measured)
  float* ws_dA;  // [Bsz*K, D, N]     per-(batch, chunk) partial dA
  float* ws_dD;  // [Bsz*K, D]        per-(batch, chunk) partial dD
  float* ws_db;  // [Bsz*K, D]        per-(batch, chunk) partial ddelta_bias
  int64_t K, Lc;
  int64_t nDblk;   // G * nJ: 64-channel blocks per batch
  int64_t nJ;      // ceil(Dg / 64)
  int64_t nsg;     // state groups of 16 (1 when dstate <= 16)
  int64_t NPr;     // row width of the dB / dC partials (16 * nsg, zero-padded)
  int32_t has_D, has_z, has_bias, softplus;
  int32_t rowvec;  // 1: whole 8-step row blocks per lane (Row8; last, so the other fields keep
                   // the offsets the kernels were measured with)
};

// States per group of the backward kernels (a dstate above it is split into groups).
constexpr int kBwdGroup = 16;

// Parameter block of the inter-chunk carry kernels.
struct CarryK {
  const float* A; int64_t sA[2];
  float* ws;             // [nch, K, N] summaries in, carried values out
  const float* ws_s;     // [nch, K] sum of Delta per chunk
  const int32_t* ws_r;   // [nch, K] 1 when a sequence starts inside the chunk; NULL: none do
  int64_t nch, D, K, N;
};

// Parameter block of the causal conv1d kernels (strides in elements).
struct ConvK {
  int64_t Bsz, D, L;
  int64_t sx[3], so[3], sdo[3], sdx[3];
  int64_t sw[2], sb, sdw[2], sdb;
  const void* x; const float* w; const float* bias; void* out;
  const void* dout; void* dx; float* dw; float* dbias;
  float* ws;        // backward: [Bsz * nsplit, D, W + 1] per-block dweight | dbias partials
  float* ws2;       // backward: [nslice, D, W + 1] sums of the partial rows per row slice
  int64_t nslice, rps;  // backward: row slices of the partials, rows per slice
  int64_t T;        // steps per wave tile
  int64_t nCb;      // channel blocks (64 lanes x VEC channels)
  int64_t ntile4;   // blocks of 4 wave tiles along the sequence
  int64_t nsplit;   // backward: blocks per (batch, channel block) along the sequence
  int64_t tps;      // backward: tile blocks per split
};

// Loads / stores of one element whose dtype is a wave-uniform runtime value.
__device__ inline float load_any(const void* p, int64_t i, int dt) {
  if (dt == S6_F32) return Elem<float>::load(p, i);
  if (dt == S6_BF16) return Elem<bf16>::load(p, i);
  return Elem<f16>::load(p, i);
}

__device__ inline void store_any(void* p, int64_t i, float v, int dt) {
  if (dt == S6_F32) Elem<float>::store(p, i, v);
  else if (dt == S6_BF16) Elem<bf16>::store(p, i, v);
  else Elem<f16>::store(p, i, v);
}

// Parameter block of the Mamba-2 SSD kernels (strides in elements).
struct SsdK {
  int64_t Bsz, L, H, P, G, N, Q, K;   // K = number of chunks of Q steps
  int64_t Pa, Na;  // headdim and dstate of the caller's tensors; P, N: the kernels' tile sizes
                   // (Pa <= P, Na <= N; x, z, B, C, dout are then zero-padded copies)
  int64_t hpg;                        // heads per B / C group
  int32_t io;                         // dtype of x, z, B, C, dt, out
  int32_t softplus, has_bias, has_D, D_hdim, has_z, has_init, has_seq;
  float dt_min, dt_max;
  const void* x; int64_t sx[4];
  const void* dt; int64_t sdt[3];
  const float* A; int64_t sA;
  const void* Bm; int64_t sB[4];
  const void* Cm; int64_t sC[4];
  const float* Dp; int64_t sD[2];
  const void* z; int64_t sz[4];
  const float* bias; int64_t sbias;
  const float* init; int64_t sinit[4];
  const int32_t* seq; int64_t sseq[2];
  void* out; int64_t sout[4];
  void* out_x; int64_t soutx[4];      // NULL: not written
  float* final_states;                // NULL: not written
  float* dtq;   // [Bsz, H, K, Q] processed dt (0 past the sequence end)
  float* dacs;  // [Bsz, H, K, Q] cumulative dt * A within each chunk
  float* st;    // [Bsz, K, H, P, N] chunk states
  void* hs;     // [Bsz, K, H, P, N] state entering each chunk (io dtype)
  float* cb;    // [Bsz, K, G, Q, Q] C B^T within each chunk (lower-triangle tiles written)
  const int32_t* cu; int64_t nseq;    // varlen states: sequence bounds (batch 1)
  void* vst;                          // [nseq, H, P, N] io dtype; NULL: not written
  // ---- backward only ----
  const void* dout; int64_t sdout[4];
  const void* dy; int64_t sdy[4];     // dout * silu(z) (workspace) or dout itself
  void* dyw;                          // [Bsz, L, H, P] io workspace for dy when z is given
  void* dz; int64_t sdz[4];
  void* dx; int64_t sdx[4];
  void* ddt; int64_t sddt[3];
  void* dBo; int64_t sdBo[4];
  void* dCo; int64_t sdCo[4];
  float* dA; float* dD; float* ddt_bias; float* dinit;   // dinit: [Bsz, H, P, N] contiguous
  const float* dfinal; int64_t sdfinal[4];
  float* dhl;     // [Bsz, K, H, P, N] gradient of each chunk's entering state from its outputs
  void* dst;      // [Bsz, K, H, P, N] io: gradient of each chunk state
  float* ddal;    // [Bsz, H, K, nE] partial gradients of S_last through the state passing
  int64_t nE;     // element blocks of the state passing backward
  float* ddtd;    // [Bsz, H, K, Q] direct dt gradient (x . (T1 + T2))
  float* dDp;     // [Bsz * K * Q/64, H(, P)] partial dD
  float* qv;      // [N / min(N, 64), Bsz, H, K, Q] chunk-state decay terms, per dstate slice
  float* uv;      // [N / min(N, 64), Bsz, H, K, Q] inter-chunk decay terms, per dstate slice
  float* dBp;     // [Bsz, L, G, N] fp32 dB from the chunk states
  float* dCp;     // [Bsz, L, G, N] fp32 dC from the entering states
  float* dcb;     // [Bsz, K, G, Q, Q] gradient of C B^T (lower-triangle tiles)
  float* rs;      // [Q/64, Bsz, H, K, Q] row sums of the intra-chunk decay terms, per column tile
  float* csp;     // [Bsz, H, K, Q/64, Q] column-sum partials per row tile
  float* dAp;     // [Bsz * K, H] partial dA
  float* dbp;     // [Bsz * K, H] partial ddt_bias
};

// Parameter block of the selective_state_update kernel (strides in elements).
struct SsuK {
  int64_t batch, nheads, dim, dstate, hpg;   // hpg: heads per B / C group
  int32_t io, bc;                            // dtypes of x / dt / z / out and of B / C
  void* state; int64_t ss[4];
  const void* x; int64_t sx[3];
  const void* dt; int64_t sdt[3];
  const float* bias; int64_t sbias[2];       // NULL: no dt_bias
  const float* A; int64_t sA[3];
  const void* B; int64_t sB[3];
  const void* C; int64_t sC[3];
  const float* Dp; int64_t sD[2];            // NULL: no D
  const void* z; int64_t sz[3];              // NULL: no z
  void* out; int64_t so[3];
  int32_t a_vec, bc_vec;   // row kernel: A / B and C rows contiguous and 4-element aligned
};

inline hipError_t record_event(void* const* ev, int i, hipStream_t st) {
  if (ev == nullptr || ev[i] == nullptr) return hipSuccess;
  return hipEventRecord((hipEvent_t)ev[i], st);
}

// Per input dtype (one translation unit each): the dtype-templated scan kernels.
template <typename Tio>
hipError_t launch_fwd_io(const FwdK& k, int bc_dtype, hipStream_t st, void* const* ev);
template <typename Tio>
hipError_t launch_bwd_io(const BwdK& k, int bc_dtype, hipStream_t st, void* const* ev);
template <typename Tio>
hipError_t launch_fwd_lanes_io(const FwdK& k, int bc_dtype, hipStream_t st, void* const* ev);
template <typename Tio>
hipError_t launch_fwd_rowvec_io(const FwdK& k, int bc_dtype, hipStream_t st, void* const* ev);
template <typename Tio>
hipError_t launch_bwd_rowvec_io(const BwdK& k, int bc_dtype, hipStream_t st, void* const* ev);

// s6_misc.hip: carries, reductions, fills, B/C relayout.
hipError_t launch_fwd_carry(const FwdK& k, hipStream_t st);
hipError_t launch_bwd_carry(const BwdK& k, hipStream_t st);
hipError_t launch_bwd_reduce(const BwdK& k, hipStream_t st);

// ev (nullable): hipEvent_t pair recorded around the main scan kernel.
hipError_t launch_fwd(const FwdK& k, int io_dtype, int bc_dtype, hipStream_t st, void* const* ev);
hipError_t launch_bwd(const BwdK& k, int io_dtype, int bc_dtype, hipStream_t st, void* const* ev);
// s6_conv.hip: causal conv1d.  vec: channels per lane (1 = any strides).
hipError_t launch_conv_fwd(const ConvK& k, int io_dtype, int width, int vec, bool silu,
                           hipStream_t st);
hipError_t launch_conv_bwd(const ConvK& k, int io_dtype, int width, int vec, bool silu,
                           hipStream_t st);
// s6_ssd.hip: the Mamba-2 SSD forward; prep = dt processing, chunk states, state passing
// and C B^T (shared with the backward, which recomputes them); dstates = the chunk-state
// kernel in its backward mode (gradient of each chunk's entering state).
hipError_t launch_ssd_fwd(const SsdK& k, hipStream_t st, void* const* ev = nullptr);
hipError_t launch_ssd_prep(const SsdK& k, hipStream_t st);
hipError_t launch_ssd_dstates(const SsdK& k, hipStream_t st);
// s6_ssd_bwd.hip: the Mamba-2 SSD backward.
hipError_t launch_ssd_bwd(const SsdK& k, hipStream_t st);
// s6_ssu.hip: one decode step of the state.
// rows: the state and A rows are contiguous and 16-byte aligned (vectorised row mapping).
hipError_t launch_state_update(const SsuK& k, int state_dtype, bool softplus, bool rows,
                               hipStream_t st);
hipError_t launch_fill(float* p, int64_t n, float v, hipStream_t st);
// dst[i] = src[i] for every 4-D index i inside ddim, 0 where i lies outside sdim (strides in
// elements, esize 2 or 4): zero-pads a tensor into a larger buffer, or copies the leading part
// of a padded buffer out.
hipError_t launch_copy4d(const void* src, const int64_t ss[4], const int64_t sdim[4], void* dst,
                         const int64_t ds[4], const int64_t ddim[4], int esize, hipStream_t st);
hipError_t launch_relayout(const void* src, const int64_t s[4], int esize, void* dst,
                           int64_t Bsz, int64_t G, int64_t N, int64_t NP, int64_t L,
                           hipStream_t st);

}  // namespace s6
