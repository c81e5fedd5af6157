// Internal launch interface between the C ABI (s6_abi.cpp) and the HIP kernels.
#pragma once
#include "s6_common.h"

namespace s6 {

// Parameter block of the backward kernels (strides in elements).
struct BwdK {
  int64_t Bsz, D, L, N, G;
  int64_t su[3], sdl[3], sz[3], sdo[3], sout[3], sdu[3], sddl[3], sdz[3];
  int64_t sA[2], sD, sbias;
  int64_t sB[4], sC[4];
  int64_t sdA[2], sdD, sdbias;
  int64_t sdB[4], sdC[4];
  const void* u; const void* delta; const void* z; const void* dout; const void* out;
  const float* A; const float* Dp; const float* bias;
  const void* Bm; const void* Cm;
  const int32_t* cu; int32_t nseq;
  const float* x_ckpt; int64_t nck;
  void* du; void* ddelta; void* dz;
  float* dA; float* dD; float* dbias; float* dB; float* dC;
  float* ws_g;   // [Bsz*D, K, N]  reverse chunk summaries, then carried-in gradients
  float* ws_s;   // [Bsz*D, K]     sum of Delta over each chunk
  float* ws_pB;  // [Bsz, G, nJ4, L, N]  per-channel-block partial dB
  float* ws_pC;  // [Bsz, G, nJ4, L, N]  per-channel-block partial dC
  int64_t K, Lc;
  int64_t nDblk;   // G * ceil(Dg / 64)   (summary kernel, 64-channel blocks)
  int64_t nJ4;     // ceil(Dg / 256)      (main kernel, 256-channel blocks per group)
  int32_t has_D, has_z, has_bias, softplus;
};

// ev (nullable): hipEvent_t pair recorded around the main scan kernel.
hipError_t launch_fwd(const FwdK& k, int io_dtype, int bc_dtype, hipStream_t st, void* const* ev);
hipError_t launch_bwd(const BwdK& k, int io_dtype, int bc_dtype, hipStream_t st, void* const* ev);
hipError_t launch_fill(float* p, int64_t n, float v, hipStream_t st);
hipError_t launch_relayout(const void* src, const int64_t s[4], int esize, void* dst,
                           int64_t Bsz, int64_t G, int64_t N, int64_t NP, int64_t L,
                           hipStream_t st);

}  // namespace s6
