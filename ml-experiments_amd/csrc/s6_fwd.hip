// Forward S6 selective scan for gfx950.
//
// Mapping: one lane owns one channel (b, d) and keeps all of its N states in VGPRs; a
// 64-lane workgroup covers 64 channels of one (batch, group).  B_t and C_t are identical
// for every lane of the workgroup, so they are read through the scalar cache into SGPRs
// and feed v_fma directly.  The sequence is cut into K chunks of Lc steps so that
// B * D / 64 * K waves fill the chip:
//   fwd_scan<MODE=0>   chunk summary: state of each chunk from a zero start and the sum of
//                      Delta since its last sequence start                 (chunks 0..K-2)
//   fwd_carry          segmented prefix over chunks, h_in(c+1) = exp(A S_c) h_in(c) + h_loc(c),
//                      as a 64-lane parallel scan (one wave per channel)
//   fwd_scan<MODE=1,2> rescan of each chunk from its carried-in state, fused with
//                      y = C h + D u, the silu(z) gate (MODE 2), checkpoints and last states.
// The recurrence and its rounding points follow selective_scan_ref
// (selective_scan_interface.py:107-156): Delta = softplus(delta + bias) in fp32,
// abar = exp(Delta * A), h = abar * h + Delta * u * B, y = sum_n C h + D u.
#include <type_traits>

#include "s6_internal.h"

namespace s6 {

// MODE 0: chunk summary; 1: output pass; 2: output pass with the silu(z) gate.
// DTM: how Delta is formed from the delta input (kDtRaw / kDtBias / kDtSoftplus).
// MULTI (dstate > 32): the workgroup holds one wave per group of NS = 16 states (p.nsg
// waves) of the same 64 channels and chunk.  The state groups scan independently; in the
// output pass each wave's share of y (its states' C h) goes through LDS once per 8-step
// block, and the waves then split the block's steps to sum the groups in a fixed order, add
// D u, gate and store.  This keeps every wave at the register footprint of 16 states; at
// 17-32 states one wave holding them all measured faster (2 groups do not pay for the
// duplicated per-step work and the barrier).
// Occupancy target: 4 waves per SIMD (<= 128 VGPRs) for MULTI and for the z-gated softplus
// output pass at 16 states, which the compiler otherwise lays out at 129 VGPRs (3 waves;
// measured 5% slower).  The raw / bias z-gated variants would spill at 128 and keep the
// default.
// VEC (p.rowvec; not with MULTI): u / delta / z / out / out_z have a contiguous time axis,
// 16-byte aligned at every block of 8 steps, and every chunk is whole blocks; each lane then
// moves a block of its row with one 16-byte access per tensor (Row8) instead of eight, each of
// which would touch one cache line per lane (measured: the cfg3-shape forward with
// checkpoints 1.00 -> 0.64 ms, the z-gated softplus forward at B32 L4096 D256 1.13 -> 0.51 ms,
// both on [B, D, L] L-contiguous inputs).
template <typename Tio, typename Tbc, int NS, int MODE, int DTM, bool MULTI, bool VEC>
__global__ void __launch_bounds__(MULTI ? 4 * kWave : kWave)
    __attribute__((amdgpu_waves_per_eu((MULTI || (MODE == 2 && DTM == kDtSoftplus && NS <= 16)) ? 4 : 1)))
    fwd_scan(FwdK p) {
  constexpr bool FULL = MODE != 0;
  constexpr bool HAS_Z = MODE == 2;
  constexpr int TB = kCk;  // steps per unrolled block = checkpoint interval
  constexpr int ES = Elem<Tio>::kSize;
  constexpr int EB = Elem<Tbc>::kSize;
  constexpr int GS = NS < kGroupStates<Tbc> ? NS : kGroupStates<Tbc>;  // states per scalar group
  constexpr int NG = NS / GS;
  static_assert(!MULTI || NS == 16, "state groups of 16");
  static_assert(!(MULTI && VEC), "row vectors with one wave per channel block only");
  const int lane = threadIdx.x & (kWave - 1);
  // State group of this wave, made wave-uniform (an SGPR) so that the B / C row addresses
  // derived from it stay scalar and their loads stay on the scalar cache.
  const int gn = MULTI ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave)) : 0;
  const int s0 = gn * NS;                                   // its first state
  // MULTI output pass: the groups' shares of y, [block parity][group][step][lane].
  __shared__ float ysh[2][4][TB][kWave];
  const BlockPos bp = block_pos(p.Bsz * p.nDblk);
  const int64_t Dg = p.D / p.G;
  const int64_t nJ = (Dg + kWave - 1) / kWave;
  const int64_t b = bp.x / p.nDblk;
  const int64_t rem = bp.x % p.nDblk;
  const int64_t g = rem / nJ;
  const int64_t j = rem % nJ;
  const int64_t dloc = j * kWave + lane;
  const bool active = dloc < Dg;
  const int64_t d0 = g * Dg + j * kWave;  // first channel of this wave
  const int64_t d = g * Dg + (active ? dloc : Dg - 1);
  const int c = (int)bp.y;
  const int L = (int)p.L;
  const int t0 = c * (int)p.Lc;
  const int t1 = min(t0 + (int)p.Lc, L);
  const int N = (int)p.N - s0;  // states of the group (may exceed NS)
  const int Nw = min(N, NS);     // states this wave owns
  const bool varlen = p.nseq > 0;

  float Ap[NS];
  float h[NS];
  // Prologue loads are unconditional, from in-bounds addresses (the group's last real state
  // for padded ones, A in place of an absent bias / D), and masked afterwards: a load under a
  // branch waits for itself before the branch joins, one round trip each.
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    const float a = p.A[d * p.sA[0] + (s0 + (n < N ? n : N - 1)) * p.sA[1]];
    Ap[n] = (n < N) ? a * kLog2e : 0.f;
    h[n] = 0.f;
  }
  const int64_t ch = b * p.D + d;  // channel index for workspaces
  if (FULL && c > 0) {
    const float* hin = p.ws_h + (ch * p.K + c) * p.N + s0;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const float v = hin[n < N ? n : N - 1];
      h[n] = (n < N) ? v : 0.f;
    }
  }
  const bool hb = DTM != kDtRaw && p.has_bias;
  const float bias_v = (hb ? p.bias : p.A)[hb ? d * p.sbias : 0];
  const float bias = hb ? bias_v : 0.f;
  const bool hd = FULL && p.has_D;
  const float Dv_v = (hd ? p.Dp : p.A)[hd ? d * p.sD : 0];
  const float Dv = hd ? Dv_v : 0.f;
  // checkpoints: [batch, nck, dim, dstate]
  float* const xck = (FULL && p.x_ckpt != nullptr) ? p.x_ckpt + b * p.sck[0] + d * p.sck[2] + s0 : nullptr;
  const int64_t xck_step = p.sck[1];

  // Buffer resources based at (b, d0, t0) of each [batch, dim, seqlen] tensor.
  const auto rs_u = make_rsrc((const char*)p.u + (b * p.su[0] + d0 * p.su[1] + (int64_t)t0 * p.su[2]) * ES);
  const auto rs_d = make_rsrc((const char*)p.delta + (b * p.sdl[0] + d0 * p.sdl[1] + (int64_t)t0 * p.sdl[2]) * ES);
  const uint32_t vo_u = active ? (uint32_t)(lane * p.su[1] * ES) : kOffDrop;
  const uint32_t vo_d = active ? (uint32_t)(lane * p.sdl[1] * ES) : kOffDrop;
  const uint32_t st_u = (uint32_t)(p.su[2] * ES), st_d = (uint32_t)(p.sdl[2] * ES);
  // Unused resources (no output in the summary pass, no z) point at u and are never read.
  const auto rs_o = make_rsrc(FULL ? (const char*)p.out + (b * p.so[0] + d0 * p.so[1] + (int64_t)t0 * p.so[2]) * ES
                                   : (const char*)p.u);
  const auto rs_z = make_rsrc(HAS_Z ? (const char*)p.z + (b * p.sz[0] + d0 * p.sz[1] + (int64_t)t0 * p.sz[2]) * ES
                                    : (const char*)p.u);
  const auto rs_oz = make_rsrc(HAS_Z ? (const char*)p.out_z + (b * p.soz[0] + d0 * p.soz[1] + (int64_t)t0 * p.soz[2]) * ES
                                     : (const char*)p.u);
  const uint32_t vo_o = (FULL && active) ? (uint32_t)(lane * p.so[1] * ES) : kOffDrop;
  const uint32_t vo_z = (HAS_Z && active) ? (uint32_t)(lane * p.sz[1] * ES) : kOffDrop;
  const uint32_t vo_oz = (HAS_Z && active) ? (uint32_t)(lane * p.soz[1] * ES) : kOffDrop;
  const uint32_t st_o = FULL ? (uint32_t)(p.so[2] * ES) : 0u;
  const uint32_t st_z = HAS_Z ? (uint32_t)(p.sz[2] * ES) : 0u;
  const uint32_t st_oz = HAS_Z ? (uint32_t)(p.soz[2] * ES) : 0u;
  // B / C rows of this wave's (batch, group), from step t0; 32-bit byte offsets per step.
  const char* const Bbase = (const char*)p.Bm + (b * p.sB[0] + g * p.sB[1] + (int64_t)t0 * p.sB[3] + s0) * EB;
  const char* const Cbase = (const char*)p.Cm + (b * p.sC[0] + g * p.sC[1] + (int64_t)t0 * p.sC[3] + s0) * EB;
  const uint32_t Bst = (uint32_t)(p.sB[3] * EB), Cst = (uint32_t)(p.sC[3] * EB);

  SeqCursor sc;
  sc.idx = 0;
  sc.pending = INT64_MAX;
  if (varlen) sc = seq_cursor_at(p.cu, p.nseq, t0);
  float ssum = 0.f;         // sum of Delta since the last sequence start (chunk summary only)
  bool seen_start = false;  // a sequence started inside this chunk

  // Per-step form (!VEC): a register double buffer; the next block's u / delta / z are in
  // flight, as raw bits, while the current block computes, and loads past t1 re-read step
  // t1 - 1.  Outputs and checkpoints are stored as they are computed.
  // Row-block form (VEC): a block begins by taking over its rows (loaded one block earlier),
  // then stores the previous block's outputs and checkpoint, then issues the next block's
  // loads, and its steps issue no vector memory operation.  The compiler waits for a load
  // with vmcnt(0) whenever stores are in flight, so this order makes the one wait per block,
  // at the takeover, cover only operations a block old.  (The same order in the per-step
  // form measured 3-9% slower: the held outputs cost registers there.)
  uint32_t un[VEC ? 1 : TB], dn[VEC ? 1 : TB], zn[VEC ? 1 : TB];
  Row8<Tio> vu, vd, vz;  // VEC: the next block's rows
  auto fetch = [&](int tb) {
    const uint32_t r = (uint32_t)(tb - t0);
    if constexpr (VEC) {
      vu.load(rs_u, vo_u, r * st_u);
      vd.load(rs_d, vo_d, r * st_d);
      if (HAS_Z) vz.load(rs_z, vo_z, r * st_z);
    } else {
#pragma unroll
      for (int i = 0; i < TB; ++i) {
        const uint32_t ri = (uint32_t)(min(tb + i, t1 - 1) - t0);
        un[i] = Buf<Tio>::load_raw(rs_u, vo_u, ri * st_u);
        dn[i] = Buf<Tio>::load_raw(rs_d, vo_d, ri * st_d);
        if (HAS_Z && !MULTI) zn[i] = Buf<Tio>::load_raw(rs_z, vo_z, ri * st_z);
      }
    }
  };
  fetch(t0);
  if constexpr (VEC) {
    // The loop's first use of a block's rows would otherwise inherit this load's wait, which
    // on later blocks would also cover the stores issued just before it.
    vu.settle();
    vd.settle();
    if (HAS_Z) vz.settle();
  }
  // VEC: the previous block's packed outputs, stored at the top of the next block (or after
  // the loop); h still holds the block's final state there, which is its checkpoint.
  Row8<Tio> po, poz;
  auto flush = [&](int tbp) {
    if constexpr (VEC && FULL) {
      const uint32_t r = (uint32_t)(tbp - t0);
      po.store(rs_o, vo_o, r * st_o);
      if (HAS_Z) poz.store(rs_oz, vo_oz, r * st_oz);
      if (xck != nullptr && active) store_state<NS>(xck + (int64_t)(tbp / kCk) * xck_step, h, Nw);
    }
  };

  // Scalar-cache pipeline for B_t / C_t (touch / opaque, s6_common.h): one group of GS
  // states is in flight while the previous one is consumed.
  BCGroup<Tbc> bnx, cnx;
  bnx.template load<GS>(Bbase);
  if (FULL) cnx.template load<GS>(Cbase);

  for (int tb = t0; tb < t1; tb += TB) {
    float uc[VEC ? 1 : TB], dc[VEC ? 1 : TB], zc[VEC ? 1 : TB];
    Row8<Tio> ru, rd, rz;  // VEC: this block's rows
    if constexpr (VEC) {
      ru = vu;
      rd = vd;
      if (HAS_Z) rz = vz;
      if (tb > t0) flush(tb - TB);
    } else {
#pragma unroll
      for (int i = 0; i < TB; ++i) {
        uc[i] = Buf<Tio>::from_raw(un[i]);
        dc[i] = Buf<Tio>::from_raw(dn[i]);
        zc[i] = (HAS_Z && !MULTI) ? Buf<Tio>::from_raw(zn[i]) : 0.f;
        // converted here, not where the steps use them: the raw registers then die before
        // the next block's loads reuse them, instead of being copied at the loop's back edge
        // (a copy that waits for those loads and for every store issued since)
        asm volatile("" : "+v"(uc[i]), "+v"(dc[i]));
        if constexpr (HAS_Z && !MULTI) asm volatile("" : "+v"(zc[i]));
      }
    }
    // MULTI output pass: u (and z) of the steps this wave finishes after the block,
    // i = gn + k nsg, reloaded now (they are in cache from the prefetch) so that the block's
    // own u / z registers need not live until the end of the block.
    float ucb[4] = {}, zcb[4] = {};
    if constexpr (MULTI && FULL) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = gn + k * p.nsg;
        if (i < TB) {
          const uint32_t r = (uint32_t)(min(tb + i, t1 - 1) - t0);
          ucb[k] = Buf<Tio>::load(rs_u, vo_u, r * st_u);
          if (HAS_Z) zcb[k] = Buf<Tio>::load(rs_z, vo_z, r * st_z);
        }
      }
    }
    // Unconditional (the last block re-reads itself: VEC from a clamped block, the per-step
    // form from steps clamped to t1 - 1), so that the next block's inputs are always a fresh
    // load; a skipped load would merge the old value back in, and the compiler then copies
    // the fresh one, which waits for it.
    if constexpr (VEC) fetch(min(tb + TB, t1 - TB));
    else fetch(tb + TB);
    // A sequence starts inside this block, or right after it (its predecessor's final
    // state is stored at the block's last step).
    const bool blk_has_start = varlen && sc.pending <= (int64_t)tb + TB;
    // Blocks that are full, hold no sequence boundary and do not end the input take the
    // fast path: no per-step bounds, reset or final-state checks.
    const bool general = blk_has_start || tb + TB > t1 || (FULL && tb + TB >= L);
    // VEC: the block's outputs, packed after the general / fast paths join (packed inside
    // them, the compiler keeps both paths' values apart: about 90 more VGPRs).
    float yb[TB];
    auto block = [&](auto gen_tag) {
      constexpr bool GEN = decltype(gen_tag)::value;
#pragma unroll
      for (int i = 0; i < TB; ++i) {
        const int t = tb + i;
        if (GEN && t >= t1) break;
        if (GEN && blk_has_start && t == sc.pending) {
#pragma unroll
          for (int n = 0; n < NS; ++n) h[n] = 0.f;
          ssum = 0.f;
          seen_start = true;
          while (sc.idx <= p.nseq && (int64_t)p.cu[sc.idx] <= t) ++sc.idx;
          sc.pending = (sc.idx <= p.nseq) ? (int64_t)p.cu[sc.idx] : INT64_MAX;
        }
        const uint32_t r = (uint32_t)(t - t0);
        const uint32_t rn = (uint32_t)(min(t + 1, t1 - 1) - t0);
        const float uu = VEC ? ru.get(i) : uc[VEC ? 0 : i];
        const float dt = prep_dt<DTM>(VEC ? rd.get(i) : dc[VEC ? 0 : i], bias);
        const float dtu = dt * uu;
        // y accumulates in 4 independent FMA chains (n mod 4): shorter dependency chains
        // and a smaller rounding error than one long chain.
        float ys[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          bnx.touch();
          if (FULL) cnx.touch();
          const BCGroup<Tbc> bcur = bnx;
          BCGroup<Tbc> ccur;
          if (FULL) ccur = cnx;
          const uint32_t goff = (uint32_t)((gi + 1) * GS * EB);
          const uint32_t ob = opaque(gi + 1 < NG ? r * Bst + goff : rn * Bst);
          bnx.template load<GS>(Bbase + ob);
          if (FULL) cnx.template load<GS>(Cbase + opaque(gi + 1 < NG ? r * Cst + goff : rn * Cst));
#pragma unroll
          for (int k = 0; k < GS; ++k) {
            const int n = gi * GS + k;
            const float a = fast_exp2(dt * Ap[n]);
            h[n] = fmaf(a, h[n], dtu * bcur.get(k));
            if (FULL) ys[k & 3] = (gi == 0 && k < 4) ? ccur.get(k) * h[n] : fmaf(ccur.get(k), h[n], ys[k & 3]);
          }
        }
        if (!FULL) {
          ssum += dt;
        } else {
          float y = (ys[0] + ys[1]) + (ys[2] + ys[3]);
          if constexpr (MULTI) {
            ysh[((tb - t0) / TB) & 1][gn][i][lane] = y;  // this group's share of y
          } else if constexpr (VEC) {
            yb[i] = fmaf(uu, Dv, y);
          } else {
            y = fmaf(uu, Dv, y);
            Buf<Tio>::store(rs_o, vo_o, r * st_o, y);
            if (HAS_Z) {
              const float zz = zc[VEC ? 0 : i];
              Buf<Tio>::store(rs_oz, vo_oz, r * st_oz, y * zz * sigmoidf_(zz));
            }
          }
          if (GEN) {
            // Final states: of the sequence that owns step t when the next step starts a
            // new one (the end of the input included), else of the batch row at its last
            // step.  The wave-uniform conditions are tested before the per-lane one.
            const bool seq_end = varlen ? (blk_has_start && t + 1 == sc.pending) : (t == L - 1);
            if (seq_end && p.last_state != nullptr) {
              // Sequence row of the final state; a row outside [0, nseq) can only come
              // from offsets the host validation rejects, and is never stored.
              const int64_t row = varlen ? (int64_t)(sc.idx - 1) : b;
              const bool row_ok = !varlen || (row >= 0 && row < p.nseq);
              if (active && row_ok) store_state<NS>(p.last_state + (row * p.D + d) * p.N + s0, h, Nw);
            }
          }
          if (!VEC && (i == TB - 1 || (GEN && t == L - 1)) && xck != nullptr) {
            if (active) store_state<NS>(xck + (int64_t)(t / kCk) * xck_step, h, Nw);
          }
        }
      }
      if constexpr (MULTI && FULL) {
        // y of the block's steps: every wave wrote its share to LDS above (double-buffered
        // by block parity, so one barrier per block suffices); wave gn now finishes the
        // steps i = gn, gn + nsg, ...: groups summed in order 0..nsg-1, D u, gate, store.
        const int par = ((tb - t0) / TB) & 1;
        __syncthreads();
        const int nsg = p.nsg;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int i = gn + k * nsg;
          const int t = tb + i;
          if (i >= TB || (GEN && t >= t1)) continue;  // wave-uniform
          float y = ysh[par][0][i][lane];
#pragma unroll
          for (int q = 1; q < 4; ++q)
            if (q < nsg) y += ysh[par][q][i][lane];
          y = fmaf(ucb[k], Dv, y);
          const uint32_t r = (uint32_t)(t - t0);
          Buf<Tio>::store(rs_o, vo_o, r * st_o, y);
          if (HAS_Z) {
            const float zz = zcb[k];
            Buf<Tio>::store(rs_oz, vo_oz, r * st_oz, y * zz * sigmoidf_(zz));
          }
        }
      }
    };
    if (general) block(std::true_type{}); else block(std::false_type{});
    if constexpr (VEC && FULL) {
      po.pack(yb);
      if constexpr (HAS_Z) {
#pragma unroll
        for (int i = 0; i < TB; ++i) {
          const float zz = rz.get(i);
          yb[i] = yb[i] * zz * sigmoidf_(zz);
        }
        poz.pack(yb);
      }
    }
  }
  if constexpr (VEC) flush(t1 - TB);
  if (!FULL && active) {
    store_state<NS>(p.ws_h + (ch * p.K + c) * p.N + s0, h, Nw);
    if (gn == 0) {
      p.ws_s[ch * p.K + c] = ssum;
      if (varlen) p.ws_r[ch * p.K + c] = seen_start ? 1 : 0;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Host-side launch helpers.  The translation unit is compiled twice per input dtype: with
// S6_FWD_VEC=1 it instantiates the row-vector kernels (VEC) and defines
// launch_fwd_rowvec_io, otherwise the per-step kernels and launch_fwd_io, which routes
// row-vector problems to the other unit.
// ---------------------------------------------------------------------------------------

#ifndef S6_FWD_VEC
#define S6_FWD_VEC 0
#endif
constexpr bool kVec = S6_FWD_VEC != 0;

template <typename Tio, typename Tbc, int NS, int DTM, bool MULTI>
static hipError_t launch_scan_pair(const FwdK& k, hipStream_t st, void* const* ev) {
  constexpr bool V = kVec && !MULTI;
  hipError_t e = hipSuccess;
  const dim3 grid = xcd_grid(k.Bsz * k.nDblk, k.K);
  const dim3 block(MULTI ? (unsigned)(k.nsg * kWave) : (unsigned)kWave);
  if (k.K > 1) {
    // Summaries of chunks 0..K-2: the last chunk's summary is never used.
    const dim3 gsum = xcd_grid(k.Bsz * k.nDblk, k.K - 1);
    hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, 0, DTM, MULTI, V>), gsum, block, 0, st, k);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = launch_fwd_carry(k, st)) != hipSuccess) return e;
  }
  if ((e = record_event(ev, 0, st)) != hipSuccess) return e;
  if (k.has_z)
    hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, 2, DTM, MULTI, V>), grid, block, 0, st, k);
  else
    hipLaunchKernelGGL((fwd_scan<Tio, Tbc, NS, 1, DTM, MULTI, V>), grid, block, 0, st, k);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return record_event(ev, 1, st);
}

template <typename Tio, typename Tbc, int NS, bool MULTI>
static hipError_t launch_dt(const FwdK& k, hipStream_t st, void* const* ev) {
  switch (dt_mode(k.has_bias, k.softplus)) {
    case kDtRaw: return launch_scan_pair<Tio, Tbc, NS, kDtRaw, MULTI>(k, st, ev);
    case kDtBias: return launch_scan_pair<Tio, Tbc, NS, kDtBias, MULTI>(k, st, ev);
    default: return launch_scan_pair<Tio, Tbc, NS, kDtSoftplus, MULTI>(k, st, ev);
  }
}

template <typename Tio, typename Tbc>
static hipError_t launch_bc(const FwdK& k, hipStream_t st, void* const* ev) {
  if (k.N <= 8) return launch_dt<Tio, Tbc, 8, false>(k, st, ev);
  if (k.N <= 16) return launch_dt<Tio, Tbc, 16, false>(k, st, ev);
  if (k.N <= 32) return launch_dt<Tio, Tbc, 32, false>(k, st, ev);
  if constexpr (kVec) return hipErrorInvalidValue;  // the host routes dstate > 32 elsewhere
  else return launch_dt<Tio, Tbc, 16, true>(k, st, ev);  // k.nsg groups of 16 states
}

#if S6_FWD_VEC
template <typename Tio>
hipError_t launch_fwd_rowvec_io(const FwdK& k, int bc_dtype, hipStream_t st, void* const* ev) {
  if (bc_dtype == S6_F32) return launch_bc<Tio, float>(k, st, ev);
  return launch_bc<Tio, Tio>(k, st, ev);
}

template hipError_t launch_fwd_rowvec_io<S6_TIO>(const FwdK&, int, hipStream_t, void* const*);
#else
template <typename Tio>
hipError_t launch_fwd_io(const FwdK& k, int bc_dtype, hipStream_t st, void* const* ev) {
  if (k.lanes) return launch_fwd_lanes_io<Tio>(k, bc_dtype, st, ev);
  if (k.rowvec) return launch_fwd_rowvec_io<Tio>(k, bc_dtype, st, ev);
  // B / C are either in the input dtype or fp32 (the interface enforces it).
  if (bc_dtype == S6_F32) return launch_bc<Tio, float>(k, st, ev);
  return launch_bc<Tio, Tio>(k, st, ev);
}

template hipError_t launch_fwd_io<S6_TIO>(const FwdK&, int, hipStream_t, void* const*);
#endif

}  // namespace s6
