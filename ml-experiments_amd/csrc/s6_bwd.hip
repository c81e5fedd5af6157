// Backward S6 selective scan for gfx950.
//
// With lambda_t = dL/dh_t and g_t = abar_t lambda_t (the gradient step t passes to h_{t-1}):
//     lambda_t = C_t dy_t + g_{t+1},     g_t = abar_t lambda_t   (g_t = 0 at a sequence start)
//     q_t = abar_t h_{t-1} lambda_t   (gradient of the exponent Delta_t A)
//     dA += q Delta,  dDelta = sum_n q A + u sum_n lambda B,  du = Delta sum_n lambda B + D dy
//     dB_t += lambda Delta u,  dC_t += dy h_t        (summed over the channels of a group)
// where dy is dout, times silu(z) when z is given.  These are the gradients autograd
// produces through selective_scan_ref (selective_scan_interface.py:107-156); they replace
// the reference's native bwd (selective_scan_interface.py:67-70).
//
// Kernels (the reverse mirror of the forward's chunking; lane = channel, 64 per wave):
//   bwd_summary  per chunk c >= 1: the gradient leaving the chunk at its first step from a
//                zero inflow, and the chunk's sum of Delta.
//   bwd_carry    reverse segmented scan over chunks (s6_misc.hip): gradient entering each chunk.
//   bwd_scan     per chunk, per 8-step segment in reverse: the state saved by the forward at
//                the segment start, a forward recompute of the segment into registers, then
//                the reverse recurrence.  States are processed 8 at a time (two halves for
//                dstate 16) so the segment's states fit in VGPRs.  dB / dC are reduced over the
//                64 lanes with permlane swaps and DPP and written as one partial per wave;
//                dA / dD / ddelta_bias as one partial per (batch, chunk).
//   bwd_reduce_* fixed-order sums of the partials (s6_misc.hip): the result is deterministic.
#include <type_traits>

#include "s6_internal.h"
#include "s6_wave.h"

namespace s6 {

// VEC (p.rowvec; bwd_scan: not with MULTI): the per-channel tensors (u, delta, dout, z, out
// and du, ddelta, dz, out_z) have a contiguous time axis, 16-byte aligned at every block of 8
// steps, and every chunk is whole blocks.  Each lane then moves a block of its row with one
// 16-byte access per tensor (Row8, s6_common.h) instead of eight, each of which would touch one
// cache line per lane.  The next block's load is issued unconditionally (the first block
// re-reads itself): a skipped load would merge the old value back in, and the compiler then
// copies the fresh value right after its load, which waits for it.
template <typename Tio, typename Tbc, int NS, int DTM, bool HAS_Z, bool VEC>
__global__ void __launch_bounds__(kWave) bwd_summary(BwdK p) {
  constexpr int TB = kCk;
  constexpr int ES = Elem<Tio>::kSize;
  constexpr int EB = Elem<Tbc>::kSize;
  constexpr int GS = NS < kGroupStates<Tbc> ? NS : kGroupStates<Tbc>;
  constexpr int NG = NS / GS;
  const int lane = threadIdx.x;
  const BlockPos bp = block_pos(p.Bsz * p.nDblk);
  const int64_t Dg = p.D / p.G;
  const int64_t b = bp.x / p.nDblk;
  const int64_t rem = bp.x % p.nDblk;
  const int64_t g = rem / p.nJ;
  const int64_t j = rem % p.nJ;
  const int64_t dloc = j * kWave + lane;
  const bool active = dloc < Dg;
  const int64_t d0 = g * Dg + j * kWave;
  const int64_t d = g * Dg + (active ? dloc : Dg - 1);
  const int c = 1 + (int)(bp.y % (p.K - 1));
  const int s0 = (int)(bp.y / (p.K - 1)) * NS;  // first state of this wave's state group
  const int t0 = c * (int)p.Lc;
  const int t1 = min(t0 + (int)p.Lc, (int)p.L);
  const int N = (int)p.N - s0;                   // states of the group (may exceed NS)
  const bool varlen = p.nseq > 0;

  // Prologue loads unconditional from in-bounds addresses, masked afterwards (a load under a
  // branch waits for itself before the branch joins).
  float Ap[NS], gs[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    const float a = p.A[d * p.sA[0] + (s0 + (n < N ? n : N - 1)) * p.sA[1]];
    Ap[n] = (n < N) ? a * kLog2e : 0.f;
    gs[n] = 0.f;
  }
  const bool hb = DTM != kDtRaw && p.has_bias;
  const float bias_v = (hb ? p.bias : p.A)[hb ? d * p.sbias : 0];
  const float bias = hb ? bias_v : 0.f;
  const auto rs_o = make_rsrc((const char*)p.dout + (b * p.sdo[0] + d0 * p.sdo[1] + (int64_t)t0 * p.sdo[2]) * ES);
  const auto rs_d = make_rsrc((const char*)p.delta + (b * p.sdl[0] + d0 * p.sdl[1] + (int64_t)t0 * p.sdl[2]) * ES);
  const auto rs_z = make_rsrc(HAS_Z ? (const char*)p.z + (b * p.sz[0] + d0 * p.sz[1] + (int64_t)t0 * p.sz[2]) * ES
                                    : (const char*)p.dout);
  const uint32_t vo_o = active ? (uint32_t)(lane * p.sdo[1] * ES) : kOffDrop;
  const uint32_t vo_d = active ? (uint32_t)(lane * p.sdl[1] * ES) : kOffDrop;
  const uint32_t vo_z = (HAS_Z && active) ? (uint32_t)(lane * p.sz[1] * ES) : kOffDrop;
  const uint32_t st_o = (uint32_t)(p.sdo[2] * ES), st_d = (uint32_t)(p.sdl[2] * ES);
  const uint32_t st_z = HAS_Z ? (uint32_t)(p.sz[2] * ES) : 0u;
  const char* const Cbase =
      (const char*)p.Cm + (b * p.sC[0] + g * p.sC[1] + (int64_t)t0 * p.sC[3] + s0) * EB;
  const uint32_t Cst = (uint32_t)(p.sC[3] * EB);

  uint32_t on[VEC ? 1 : TB], dn[VEC ? 1 : TB], zn[VEC ? 1 : TB];  // next block, raw bits
  Row8<Tio> vo, vd, vz;                                              // VEC: next block's rows
  auto fetch = [&](int tb) {
    if constexpr (VEC) {
      const uint32_t r = (uint32_t)(tb - t0);
      vo.load(rs_o, vo_o, r * st_o);
      vd.load(rs_d, vo_d, r * st_d);
      if (HAS_Z) vz.load(rs_z, vo_z, r * st_z);
    } else {
#pragma unroll
      for (int i = 0; i < TB; ++i) {
        const uint32_t r = (uint32_t)(min(tb + i, t1 - 1) - t0);
        on[i] = Buf<Tio>::load_raw(rs_o, vo_o, r * st_o);
        dn[i] = Buf<Tio>::load_raw(rs_d, vo_d, r * st_d);
        if (HAS_Z) zn[i] = Buf<Tio>::load_raw(rs_z, vo_z, r * st_z);
      }
    }
  };
  const int tlast = t0 + ((t1 - 1 - t0) / TB) * TB;  // first step of the last block
  fetch(tlast);
  if constexpr (VEC) {
    vo.settle();
    vd.settle();
    if (HAS_Z) vz.settle();
  }
  BCGroup<Tbc> cnx;
  cnx.template load<GS>(Cbase + (uint32_t)(t1 - 1 - t0) * Cst);
  float ssum = 0.f;
  bool seen_start = false;  // a sequence starts inside this chunk
  SeqCursorRev rc{0, -1};
  if (varlen) rc = seq_cursor_rev_at(p.cu, p.nseq, t1);

  for (int tb = tlast; tb >= t0; tb -= TB) {
    float oc[VEC ? 1 : TB], dc[VEC ? 1 : TB], zc[VEC ? 1 : TB];
    Row8<Tio> ro, rd, rz;  // VEC: this block's rows, unpacked where used
    if constexpr (VEC) {
      ro = vo;
      rd = vd;
      if (HAS_Z) rz = vz;
      fetch(max(tb - TB, t0));
    } else {
#pragma unroll
      for (int i = 0; i < TB; ++i) {
        oc[i] = Buf<Tio>::from_raw(on[i]);
        dc[i] = Buf<Tio>::from_raw(dn[i]);
        zc[i] = HAS_Z ? Buf<Tio>::from_raw(zn[i]) : 0.f;
        // converted here, so that the raw registers die before the next block's loads reuse
        // them (no back-edge copy that waits for those loads)
        asm volatile("" : "+v"(oc[i]), "+v"(dc[i]));
        if constexpr (HAS_Z) asm volatile("" : "+v"(zc[i]));
      }
      fetch(max(tb - TB, t0));  // unconditional: the first block re-reads itself
    }
    const uint32_t smask = varlen ? start_mask_rev(rc, p.cu, tb) : 0u;
    seen_start = seen_start || smask != 0u;
#pragma unroll
    for (int i = TB - 1; i >= 0; --i) {
      const int t = tb + i;
      if (t < t1) {
        float dy = VEC ? ro.get(i) : oc[VEC ? 0 : i];
        if (HAS_Z) {
          const float zz = VEC ? rz.get(i) : zc[VEC ? 0 : i];
          dy *= zz * sigmoidf_(zz);
        }
        const float dt = prep_dt<DTM>(VEC ? rd.get(i) : dc[VEC ? 0 : i], bias);
        const uint32_t r = (uint32_t)(t - t0);
        const uint32_t rn = (uint32_t)(max(t - 1, t0) - t0);
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          cnx.touch();
          const BCGroup<Tbc> ccur = cnx;
          cnx.template load<GS>(Cbase + opaque(gi + 1 < NG ? r * Cst + (uint32_t)((gi + 1) * GS * EB)
                                                            : rn * Cst));
          // A sequence start at t cuts the flow into the previous sequence (g_t = 0); the
          // uniform branch keeps the common case free of per-state selects.
          auto body = [&](auto st_tag) {
            constexpr bool ST = decltype(st_tag)::value;
#pragma unroll
            for (int k = 0; k < GS; ++k) {
              const int n = gi * GS + k;
              const float lam = fmaf(ccur.get(k), dy, gs[n]);
              gs[n] = ST ? 0.f : fast_exp2(dt * Ap[n]) * lam;
            }
          };
          if ((smask >> i) & 1u) body(std::true_type{}); else body(std::false_type{});
        }
        ssum += dt;
      }
    }
  }
  if (active) {
    const int64_t ch = b * p.D + d;
    float* go = p.ws_g + (ch * p.K + c) * p.N + s0;
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) go[n] = gs[n];
    if (s0 == 0) {
      p.ws_s[ch * p.K + c] = ssum;
      if (varlen) p.ws_r[ch * p.K + c] = seen_start ? 1 : 0;
    }
  }
}

// MULTI: dstate > 16.  The workgroup holds one wave per group of NS (16) states of the same
// channels and chunk (p.nsg waves).  After each segment the waves exchange their per-step
// sums over states (sum lambda B, sum q A) through LDS, and wave gn finishes the steps
// gn, gn + nsg, ...: groups summed in order 0..nsg-1, du, dDelta and the ddelta_bias share.
template <typename Tio, typename Tbc, int NS, int DTM, bool HAS_Z, bool MULTI, bool VEC>
__global__ void __launch_bounds__(MULTI ? 4 * kWave : kWave)
    __attribute__((amdgpu_waves_per_eu(2, 2))) bwd_scan(BwdK p) {
  static_assert(!(MULTI && VEC), "row blocks with one wave per channel block only");
  constexpr int SEG = kCk;  // steps per segment = checkpoint interval
  constexpr int HS = 8;     // states per half
  constexpr int NH = NS / HS;
  static_assert(NS % HS == 0, "dstate padding");
  constexpr int ES = Elem<Tio>::kSize;
  constexpr int EB = Elem<Tbc>::kSize;
  const int lane = threadIdx.x & (kWave - 1);
  const BlockPos bp = block_pos(p.Bsz * p.nDblk);
  const int64_t Dg = p.D / p.G;
  const int64_t b = bp.x / p.nDblk;
  const int64_t rem = bp.x % p.nDblk;
  const int64_t g = rem / p.nJ;
  const int64_t j = rem % p.nJ;
  const int64_t dloc = j * kWave + lane;
  const bool active = dloc < Dg;
  const int64_t d0 = g * Dg + j * kWave;
  const int64_t d = g * Dg + (active ? dloc : Dg - 1);
  const int c = MULTI ? (int)bp.y : (int)(bp.y % p.K);
  // State group of this wave, wave-uniform (an SGPR) so that the B / C rows stay scalar.
  const int gn = MULTI ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave)) : 0;
  const int s0 = gn * NS;  // its first state
  const int t0 = c * (int)p.Lc;
  const int t1 = min(t0 + (int)p.Lc, (int)p.L);
  const int N = (int)p.N - s0;                    // states of the group (may exceed NS)
  const int64_t ch = b * p.D + d;
  const bool varlen = p.nseq > 0;

  float Ap[NS], gs[NS], dAacc[NS];
  {
    // prologue loads unconditional from in-bounds addresses, masked afterwards (a load under
    // a branch waits for itself before the branch joins); the carried gradient exists for K > 1
    const float* gin = p.K > 1 ? p.ws_g + (ch * p.K + c) * p.N + s0 : p.A;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const int nc = n < N ? n : N - 1;
      const float a = p.A[d * p.sA[0] + (s0 + nc) * p.sA[1]];
      const float gv = gin[p.K > 1 ? nc : 0];
      Ap[n] = (n < N) ? a * kLog2e : 0.f;
      gs[n] = (n < N && p.K > 1) ? gv : 0.f;
      dAacc[n] = 0.f;
    }
  }
  const bool hb = DTM != kDtRaw && p.has_bias;
  const float bias_v = (hb ? p.bias : p.A)[hb ? d * p.sbias : 0];
  const float bias = hb ? bias_v : 0.f;
  const float Dv_v = (p.has_D ? p.Dp : p.A)[p.has_D ? d * p.sD : 0];
  const float Dv = p.has_D ? Dv_v : 0.f;
  float dDacc = 0.f, dbacc = 0.f;

  // Buffer resources based at (b, d0, t0); inactive lanes load 0 and drop their stores.
  auto rsrc = [&](const void* base, const int64_t* s) {
    return make_rsrc((const char*)base + (b * s[0] + d0 * s[1] + (int64_t)t0 * s[2]) * ES);
  };
  const auto rs_u = rsrc(p.u, p.su), rs_d = rsrc(p.delta, p.sdl), rs_o = rsrc(p.dout, p.sdo);
  const auto rs_du = rsrc(p.du, p.sdu), rs_dd = rsrc(p.ddelta, p.sddl);
  const auto rs_z = rsrc(HAS_Z ? p.z : p.u, HAS_Z ? p.sz : p.su);
  const auto rs_y = rsrc(HAS_Z ? p.out : p.u, HAS_Z ? p.sout : p.su);
  const auto rs_dz = rsrc(HAS_Z ? p.dz : p.du, HAS_Z ? p.sdz : p.sdu);
  auto voff = [&](const int64_t* s, bool on) {
    return (on && active) ? (uint32_t)(lane * s[1] * ES) : kOffDrop;
  };
  const uint32_t vo_u = voff(p.su, true), vo_d = voff(p.sdl, true), vo_o = voff(p.sdo, true);
  const uint32_t vo_du = voff(p.sdu, true), vo_dd = voff(p.sddl, true);
  const uint32_t vo_z = voff(p.sz, HAS_Z), vo_y = voff(p.sout, HAS_Z), vo_dz = voff(p.sdz, HAS_Z);
  const uint32_t st_u = (uint32_t)(p.su[2] * ES), st_d = (uint32_t)(p.sdl[2] * ES);
  const uint32_t st_o = (uint32_t)(p.sdo[2] * ES);
  const uint32_t st_du = (uint32_t)(p.sdu[2] * ES), st_dd = (uint32_t)(p.sddl[2] * ES);
  const uint32_t st_z = HAS_Z ? (uint32_t)(p.sz[2] * ES) : 0u;
  const uint32_t st_y = HAS_Z ? (uint32_t)(p.sout[2] * ES) : 0u;
  const uint32_t st_dz = HAS_Z ? (uint32_t)(p.sdz[2] * ES) : 0u;
  const bool want_oz = HAS_Z && p.out_z != nullptr;
  const auto rs_oz = rsrc(want_oz ? p.out_z : p.du, want_oz ? p.soz : p.sdu);
  const uint32_t vo_oz = voff(p.soz, want_oz);
  const uint32_t st_oz = want_oz ? (uint32_t)(p.soz[2] * ES) : 0u;

  const char* const Bbase =
      (const char*)p.Bm + (b * p.sB[0] + g * p.sB[1] + (int64_t)t0 * p.sB[3] + s0) * EB;
  const char* const Cbase =
      (const char*)p.Cm + (b * p.sC[0] + g * p.sC[1] + (int64_t)t0 * p.sC[3] + s0) * EB;
  const uint32_t Bst = (uint32_t)(p.sB[3] * EB), Cst = (uint32_t)(p.sC[3] * EB);
  float* const pBrow = p.ws_pB + ((b * p.G + g) * p.nJ + j) * p.L * p.NPr + s0;
  float* const pCrow = p.ws_pC + ((b * p.G + g) * p.nJ + j) * p.L * p.NPr + s0;
  const float* const xck = p.x_ckpt + b * p.sck[0] + d * p.sck[2] + s0;  // [b, k, d, s0:]
  const int64_t xck_step = p.sck[1];

  // The forward recompute of a segment's half hands the reverse sweep one [step][8] row per
  // step through LDS, [step][4-state quarter][lane] (each lane touches only its own entries:
  // no barrier; 16 KB per wave), read back ahead of use:
  //   LDS_A: exp(Delta A), which the reverse sweep then need not recompute;
  //   LDS_H (z-gated kernels): the recomputed states themselves, which frees the 64 VGPRs that
  //   hold them otherwise.  These kernels are at their VGPR limit (256) and recompute
  //   exp(Delta A); without LDS_H they spill, which the out_z recompute pays for.
  // The softplus kernel without z uses neither: both measured slower there.
  constexpr bool LDS_A = !HAS_Z && DTM != kDtSoftplus;
  constexpr bool LDS_H = HAS_Z;
  static_assert(HS == 8, "two float4 per step");
  constexpr int kSlice = SEG * 2 * kWave;  // float4 per wave: 16 KB
  // MULTI: one dynamic slice per wave (p.nsg * 16 KB), which also carries the per-step sums
  // the waves exchange once the segment's reverse sweeps are done.
  __shared__ float4 sa_wave[(!MULTI && (LDS_A || LDS_H)) ? kSlice : 1];
  extern __shared__ float4 sa_dyn[];
  float4* const sa = MULTI ? sa_dyn + gn * kSlice : sa_wave;

  // Per-segment inputs, double-buffered: the next (earlier) segment's loads are in flight
  // while the current one computes.
  // u / delta / dout (z, out) stay raw bits until the segment that uses them; the checkpoint
  // row is loaded unconditionally from an in-bounds row (row 0 for the first segment, the
  // group's last real state for padded ones) and masked at use, so no load waits or branches
  // in the prefetch.
  constexpr int RW = VEC ? 1 : SEG;
  uint32_t un[RW], dn[RW], on[RW], zn[RW], yn[RW];
  Row8<Tio> vu, vd, vo, vz, vy;  // VEC: the next segment's rows
  float hn[NS];
  auto fetch = [&](int ts) {
    const int te = min(ts + SEG, t1);
    if constexpr (VEC) {
      const uint32_t r = (uint32_t)(ts - t0);
      vu.load(rs_u, vo_u, r * st_u);
      vd.load(rs_d, vo_d, r * st_d);
      vo.load(rs_o, vo_o, r * st_o);
      if (HAS_Z) {
        vz.load(rs_z, vo_z, r * st_z);
        vy.load(rs_y, vo_y, r * st_y);
      }
    } else {
#pragma unroll
      for (int i = 0; i < SEG; ++i) {
        const uint32_t r = (uint32_t)(min(ts + i, te - 1) - t0);
        un[i] = Buf<Tio>::load_raw(rs_u, vo_u, r * st_u);
        dn[i] = Buf<Tio>::load_raw(rs_d, vo_d, r * st_d);
        on[i] = Buf<Tio>::load_raw(rs_o, vo_o, r * st_o);
        if (HAS_Z) {
          zn[i] = Buf<Tio>::load_raw(rs_z, vo_z, r * st_z);
          yn[i] = Buf<Tio>::load_raw(rs_y, vo_y, r * st_y);
        }
      }
    }
    // the state after step ts - 1 (used only for ts > 0: zero at the start of the input)
    const float* xc = xck + (int64_t)(ts > 0 ? ts / SEG - 1 : 0) * xck_step;
#pragma unroll
    for (int n = 0; n < NS; ++n) hn[n] = xc[n < N ? n : N - 1];
  };
  const int nseg = (t1 - t0 + SEG - 1) / SEG;
  fetch(t0 + (nseg - 1) * SEG);
  if constexpr (VEC) {
    vu.settle();
    vd.settle();
    vo.settle();
    if (HAS_Z) {
      vz.settle();
      vy.settle();
    }
  }
  SeqCursorRev rc{0, -1};  // segments are visited from the last one down
  if (varlen) rc = seq_cursor_rev_at(p.cu, p.nseq, t1);

  // Scalar-cache pipeline over half rows (HS states) of B / C, as in the forward (touch /
  // opaque, s6_common.h): consume the half row(s) in flight, issue the next, compute.
  BCGroup<Tbc> bnx, cnx;
  bnx.template load<HS>(Bbase + (uint32_t)((nseg - 1) * SEG) * Bst);

  const int nsg = MULTI ? p.nsg : 1;
  const float* const sx0 = reinterpret_cast<const float*>(sa_dyn);  // MULTI: slice of group 0
  for (int s = nseg - 1; s >= 0; --s) {
    // MULTI: every wave has read the previous segment's exchanged sums from all slices
    // before this segment's recompute writes its own slice again.
    if constexpr (MULTI) __syncthreads();
    const int ts = t0 + s * SEG;
    const int te = min(ts + SEG, t1);
    float uu[SEG], dt[SEG], dy[SEG], pre[SEG], hst[NS];
    Row8<Tio> cu, cd, co, cz, cy;  // VEC: this segment's rows
    if constexpr (VEC) {
      cu = vu;
      cd = vd;
      co = vo;
      if (HAS_Z) {
        cz = vz;
        cy = vy;
      }
    }
    float dzv[SEG], ozv[SEG];  // VEC: the gate's gradient and out_z, stored as row blocks
#pragma unroll
    for (int i = 0; i < SEG; ++i) {
      const float dl = VEC ? cd.get(i) : Buf<Tio>::from_raw(dn[VEC ? 0 : i]);
      const float oo = VEC ? co.get(i) : Buf<Tio>::from_raw(on[VEC ? 0 : i]);
      uu[i] = VEC ? cu.get(i) : Buf<Tio>::from_raw(un[VEC ? 0 : i]);
      pre[i] = dl + bias;
      dt[i] = prep_dt<DTM>(dl, bias);
      dy[i] = oo;
      if (HAS_Z) {
        // out_z = out * silu(z):  dy = dout silu(z),  dz = dout out sig (1 + z (1 - sig))
        const float zz = VEC ? cz.get(i) : Buf<Tio>::from_raw(zn[VEC ? 0 : i]);
        const float yy = VEC ? cy.get(i) : Buf<Tio>::from_raw(yn[VEC ? 0 : i]);
        const float sg = sigmoidf_(zz);
        dy[i] = oo * (zz * sg);
        const float dzi = oo * yy * sg * (1.f + zz * (1.f - sg));
        const float ozi = yy * (zz * sg);
        if constexpr (VEC) {
          dzv[i] = dzi;
          ozv[i] = ozi;
        } else if (ts + i < te && gn == 0) {
          Buf<Tio>::store(rs_dz, vo_dz, (uint32_t)(ts + i - t0) * st_dz, dzi);
          if (want_oz) Buf<Tio>::store(rs_oz, vo_oz, (uint32_t)(ts + i - t0) * st_oz, ozi);
        }
      }
    }
    if constexpr (VEC && HAS_Z) {
      Row8<Tio> pz;
      pz.pack(dzv);
      pz.store(rs_dz, vo_dz, (uint32_t)(ts - t0) * st_dz);
      if (want_oz) {
        pz.pack(ozv);
        pz.store(rs_oz, vo_oz, (uint32_t)(ts - t0) * st_oz);
      }
    }
#pragma unroll
    for (int n = 0; n < NS; ++n) hst[n] = (ts > 0 && n < N) ? hn[n] : 0.f;
    // unconditional in both forms (the first segment re-reads itself), so that the next
    // segment's registers are always a fresh load and need no back-edge copy
    fetch(max(ts - SEG, t0));
    const uint32_t smask = varlen ? start_mask_rev(rc, p.cu, ts) : 0u;
    float s1[SEG], s2[SEG];
#pragma unroll
    for (int i = 0; i < SEG; ++i) s1[i] = s2[i] = 0.f;

#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      const uint32_t hoff = (uint32_t)(hh * HS * EB);
      // Forward recompute of this half's states over the segment.
      float hs[SEG][HS];
      {
        float h[HS];
#pragma unroll
        for (int k = 0; k < HS; ++k) h[k] = hst[hh * HS + k];
#pragma unroll
        for (int i = 0; i < SEG; ++i) {
          // The B / C rotation runs at every step, past the end of a partial segment too
          // (from clamped rows, unused there), so that no branch join has to merge the
          // SGPR groups; only the arithmetic is per-step conditional.
          bnx.touch();
          const BCGroup<Tbc> bcur = bnx;
          if (i + 1 < SEG) {
            bnx.template load<HS>(Bbase + opaque((uint32_t)(min(ts + i + 1, te - 1) - t0) * Bst + hoff));
          } else {  // first step of the reverse sweep
            bnx.template load<HS>(Bbase + opaque((uint32_t)(te - 1 - t0) * Bst + hoff));
            cnx.template load<HS>(Cbase + opaque((uint32_t)(te - 1 - t0) * Cst + hoff));
          }
          if (ts + i < te) {
            const float dtu = dt[i] * uu[i];
            auto body = [&](auto st_tag) {  // ST: a sequence starts at this step, h_{t-1} = 0
              constexpr bool ST = decltype(st_tag)::value;
              float av[HS];
#pragma unroll
              for (int k = 0; k < HS; ++k) {
                const float b_ = dtu * bcur.get(k);
                av[k] = ST ? 0.f : fast_exp2(dt[i] * Ap[hh * HS + k]);
                h[k] = ST ? b_ : fmaf(av[k], h[k], b_);
                hs[i][k] = h[k];
              }
              if constexpr (LDS_A && !ST) {
                sa[(i * 2) * kWave + lane] = make_float4(av[0], av[1], av[2], av[3]);
                sa[(i * 2 + 1) * kWave + lane] = make_float4(av[4], av[5], av[6], av[7]);
              }
              if constexpr (LDS_H) {
                sa[(i * 2) * kWave + lane] = make_float4(h[0], h[1], h[2], h[3]);
                sa[(i * 2 + 1) * kWave + lane] = make_float4(h[4], h[5], h[6], h[7]);
              }
            };
            if ((smask >> i) & 1u) body(std::true_type{}); else body(std::false_type{});
          }
        }
      }
      // Reverse sweep.  The LDS rows come back ahead of their use: row i - 1 (LDS_A) or
      // row i - 2 (LDS_H, which also needs row i - 1 at step i).
      float4 c_lo{}, c_hi{}, p_lo{}, p_hi{};  // rows of steps i and (LDS_H) i - 1
      if constexpr (LDS_A || LDS_H) {
        c_lo = sa[((SEG - 1) * 2) * kWave + lane];
        c_hi = sa[((SEG - 1) * 2 + 1) * kWave + lane];
      }
      if constexpr (LDS_H) {
        p_lo = sa[((SEG - 2) * 2) * kWave + lane];
        p_hi = sa[((SEG - 2) * 2 + 1) * kWave + lane];
      }
#pragma unroll
      for (int i = SEG - 1; i >= 0; --i) {
        const int t = ts + i;
        // Step i's rows as the recompute stored them (garbage at a sequence start or past the
        // input's end, where they are not used); the next read goes out now, whether or not
        // this step is inside the input, so step i always gets row i.
        const float rc[HS] = {c_lo.x, c_lo.y, c_lo.z, c_lo.w, c_hi.x, c_hi.y, c_hi.z, c_hi.w};
        const float rp[HS] = {p_lo.x, p_lo.y, p_lo.z, p_lo.w, p_hi.x, p_hi.y, p_hi.z, p_hi.w};
        if constexpr (LDS_A) {
          if (i > 0) {
            c_lo = sa[((i - 1) * 2) * kWave + lane];
            c_hi = sa[((i - 1) * 2 + 1) * kWave + lane];
          }
        }
        if constexpr (LDS_H) {
          c_lo = p_lo;
          c_hi = p_hi;
          if (i > 1) {
            p_lo = sa[((i - 2) * 2) * kWave + lane];
            p_hi = sa[((i - 2) * 2 + 1) * kWave + lane];
          }
        }
        // As in the recompute, the rotation is unconditional (clamped rows past the end).
        bnx.touch();
        cnx.touch();
        const BCGroup<Tbc> bcur = bnx, ccur = cnx;
        if (i > 0) {
          bnx.template load<HS>(Bbase + opaque((uint32_t)(min(t - 1, te - 1) - t0) * Bst + hoff));
          cnx.template load<HS>(Cbase + opaque((uint32_t)(min(t - 1, te - 1) - t0) * Cst + hoff));
        } else if (hh + 1 < NH) {  // next half, same segment
          bnx.template load<HS>(Bbase + opaque((uint32_t)(ts - t0) * Bst + hoff + HS * EB));
        } else {  // first half of the previous segment (the first segment re-reads its own)
          bnx.template load<HS>(Bbase + opaque((uint32_t)(max(ts - SEG, t0) - t0) * Bst));
        }
        if (t < te) {
          // Without LDS_A, Delta passes through an empty asm so that exp(Delta A) is recomputed
          // here rather than kept live from the recompute above (64 more VGPRs per lane).
          float dti = dt[i];
          if (!LDS_A) asm volatile("" : "+v"(dti));
          const float dtu = dti * uu[i];
          float pB[HS], pC[HS];
          auto body = [&](auto st_tag) {  // ST: a sequence starts at this step
            constexpr bool ST = decltype(st_tag)::value;
#pragma unroll
            for (int k = 0; k < HS; ++k) {
              const int n = hh * HS + k;
              const float lam = fmaf(ccur.get(k), dy[i], gs[n]);
              if (!ST) {
                const float hp = (i > 0) ? (LDS_H ? rp[k] : hs[i - 1][k]) : hst[n];
                const float a = LDS_A ? rc[k] : fast_exp2(dti * Ap[n]);
                const float gl = a * lam;      // g_t = abar_t lambda_t
                // q_t = g_t h_{t-1}; the recompute path keeps the product order its register
                // allocation was measured with
                const float q = LDS_A ? gl * hp : lam * (a * hp);
                dAacc[n] = fmaf(q, dti, dAacc[n]);
                s2[i] = fmaf(q, Ap[n], s2[i]);
                gs[n] = gl;
              } else {
                gs[n] = 0.f;
              }
              s1[i] = fmaf(lam, bcur.get(k), s1[i]);
              pB[k] = lam * dtu;
              pC[k] = dy[i] * (LDS_H ? rc[k] : hs[i][k]);
            }
          };
          if ((smask >> i) & 1u) body(std::true_type{}); else body(std::false_type{});
          wave_transpose_reduce8(pB, lane);
          wave_transpose_reduce8(pC, lane);
          const int nn = hh * HS + ((lane >> 3) & 7);
          if ((lane & 7) == 0 && nn < N) {
            pBrow[(int64_t)t * p.NPr + nn] = pB[0];
            pCrow[(int64_t)t * p.NPr + nn] = pC[0];
          }
        }
      }
    }
    // MULTI: this group's per-step sums over states go to the wave's own slice (its rows
    // are consumed by now); after the barrier wave gn finishes steps gn, gn + nsg, ...
    float* const sx = reinterpret_cast<float*>(sa);  // [2][SEG][kWave] at the slice start
    if constexpr (MULTI) {
#pragma unroll
      for (int i = 0; i < SEG; ++i) {
        sx[i * kWave + lane] = s1[i];
        sx[(SEG + i) * kWave + lane] = s2[i];
      }
      __syncthreads();
    }
    // Per-step outputs of the segment.  VEC: packed two steps at a time and stored as row
    // blocks after the loop (the segment is whole).
    Row8<Tio> pdu, pdd;
    float due = 0.f, dde = 0.f;
#pragma unroll
    for (int i = 0; i < SEG; ++i) {
      if (MULTI) {
        if (ts + i < te) dDacc = fmaf(dy[i], uu[i], dDacc);  // written by group 0 only
        if (i % nsg != gn) continue;  // wave-uniform
        float S1 = sx0[i * kWave + lane], S2 = sx0[(SEG + i) * kWave + lane];
        for (int q = 1; q < nsg; ++q) {
          S1 += sx0[q * (kSlice * 4) + i * kWave + lane];
          S2 += sx0[q * (kSlice * 4) + (SEG + i) * kWave + lane];
        }
        s1[i] = S1;
        s2[i] = S2;
      }
      if (VEC || ts + i < te) {
        const uint32_t r = (uint32_t)(ts + i - t0);
        const float duv = fmaf(dt[i], s1[i], Dv * dy[i]);
        float ddv = fmaf(uu[i], s1[i], s2[i] * 0.69314718055994531f);  // Ap = A log2(e)
        if (DTM == kDtSoftplus) ddv *= softplus20_grad(pre[i]);
        if constexpr (VEC) {
          if (i & 1) {
            pdu.set2(i >> 1, due, duv);
            pdd.set2(i >> 1, dde, ddv);
          } else {
            due = duv;
            dde = ddv;
          }
        } else {
          Buf<Tio>::store(rs_du, vo_du, r * st_du, duv);
          Buf<Tio>::store(rs_dd, vo_dd, r * st_dd, ddv);
        }
        if (!MULTI) dDacc = fmaf(dy[i], uu[i], dDacc);
        dbacc += ddv;
      }
    }
    if constexpr (VEC) {
      pdu.store(rs_du, vo_du, (uint32_t)(ts - t0) * st_du);
      pdd.store(rs_dd, vo_dd, (uint32_t)(ts - t0) * st_dd);
    }
  }
  // MULTI: the ddelta_bias shares of the groups' steps, summed by group 0 in group order.
  if constexpr (MULTI) {
    if (p.has_bias) {
      __syncthreads();
      reinterpret_cast<float*>(sa)[lane] = dbacc;
      __syncthreads();
      if (gn == 0) {
        for (int q = 1; q < nsg; ++q) dbacc += sx0[q * (kSlice * 4) + lane];
      }
    }
  }
  if (active) {
    const int64_t row = b * p.K + c;
    float* dAp = p.ws_dA + (row * p.D + d) * p.N + s0;
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) dAp[n] = dAacc[n];
    if (p.has_D && gn == 0) p.ws_dD[row * p.D + d] = dDacc;
    if (p.has_bias && gn == 0) p.ws_db[row * p.D + d] = dbacc;
  }
}

// ---------------------------------------------------------------------------------------

// The translation unit is compiled twice per input dtype: with S6_BWD_VEC=1 it instantiates
// the row-block kernels (VEC) and defines launch_bwd_rowvec_io, otherwise the per-step
// kernels and launch_bwd_io, which routes row-block problems to the other unit.
#ifndef S6_BWD_VEC
#define S6_BWD_VEC 0
#endif
constexpr bool kVec = S6_BWD_VEC != 0;

template <typename Tio, typename Tbc, int NS, int DTM, bool HAS_Z, bool MULTI>
static hipError_t launch_bwd_t(const BwdK& k, hipStream_t st, void* const* ev) {
  constexpr bool V = kVec && !MULTI;
  hipError_t e;
  const int64_t nx = k.Bsz * k.nDblk;
  if (k.K > 1) {
    hipLaunchKernelGGL((bwd_summary<Tio, Tbc, NS, DTM, HAS_Z, V>), xcd_grid(nx, (k.K - 1) * k.nsg),
                       dim3(kWave), 0, st, k);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = launch_bwd_carry(k, st)) != hipSuccess) return e;
  }
  if ((e = record_event(ev, 0, st)) != hipSuccess) return e;
  if (MULTI) {  // one workgroup of nsg waves per chunk, 16 KB of LDS per wave
    hipLaunchKernelGGL((bwd_scan<Tio, Tbc, NS, DTM, HAS_Z, MULTI, V>), xcd_grid(nx, k.K),
                       dim3((unsigned)(k.nsg * kWave)), (unsigned)(k.nsg * kCk * 2 * kWave * 16), st, k);
  } else {
    hipLaunchKernelGGL((bwd_scan<Tio, Tbc, NS, DTM, HAS_Z, MULTI, V>), xcd_grid(nx, k.K),
                       dim3(kWave), 0, st, k);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = record_event(ev, 1, st)) != hipSuccess) return e;
  return launch_bwd_reduce(k, st);
}

template <typename Tio, typename Tbc, int NS, int DTM, bool MULTI>
static hipError_t launch_bwd_z(const BwdK& k, hipStream_t st, void* const* ev) {
  return k.has_z ? launch_bwd_t<Tio, Tbc, NS, DTM, true, MULTI>(k, st, ev)
                 : launch_bwd_t<Tio, Tbc, NS, DTM, false, MULTI>(k, st, ev);
}

template <typename Tio, typename Tbc, int NS, bool MULTI>
static hipError_t launch_bwd_dt(const BwdK& k, hipStream_t st, void* const* ev) {
  switch (dt_mode(k.has_bias, k.softplus)) {
    case kDtRaw: return launch_bwd_z<Tio, Tbc, NS, kDtRaw, MULTI>(k, st, ev);
    case kDtBias: return launch_bwd_z<Tio, Tbc, NS, kDtBias, MULTI>(k, st, ev);
    default: return launch_bwd_z<Tio, Tbc, NS, kDtSoftplus, MULTI>(k, st, ev);
  }
}

template <typename Tio, typename Tbc>
static hipError_t launch_bwd_bc(const BwdK& k, hipStream_t st, void* const* ev) {
  if (k.N <= 8) return launch_bwd_dt<Tio, Tbc, 8, false>(k, st, ev);
  if (k.N <= 16) return launch_bwd_dt<Tio, Tbc, 16, false>(k, st, ev);
  if constexpr (kVec) return hipErrorInvalidValue;  // the host routes dstate > 16 elsewhere
  else return launch_bwd_dt<Tio, Tbc, 16, true>(k, st, ev);
}

#if S6_BWD_VEC
template <typename Tio>
hipError_t launch_bwd_rowvec_io(const BwdK& k, int bc_dtype, hipStream_t st, void* const* ev) {
  if (bc_dtype == S6_F32) return launch_bwd_bc<Tio, float>(k, st, ev);
  return launch_bwd_bc<Tio, Tio>(k, st, ev);
}

template hipError_t launch_bwd_rowvec_io<S6_TIO>(const BwdK&, int, hipStream_t, void* const*);
#else
template <typename Tio>
hipError_t launch_bwd_io(const BwdK& k, int bc_dtype, hipStream_t st, void* const* ev) {
  if (k.rowvec) return launch_bwd_rowvec_io<Tio>(k, bc_dtype, st, ev);
  if (bc_dtype == S6_F32) return launch_bwd_bc<Tio, float>(k, st, ev);
  return launch_bwd_bc<Tio, Tio>(k, st, ev);
}

template hipError_t launch_bwd_io<S6_TIO>(const BwdK&, int, hipStream_t, void* const*);
#endif

}  // namespace s6
