/*
 * s6scan Mamba-2 SSD (chunked state-space duality scan) -- MI355X (gfx950), C ABI.
 *
 * Replaces the Triton kernels behind `mamba_chunk_scan_combined`
 * (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/ssd_combined.py:281-332
 * forward, :563-582 entry point; kernels in ssd_chunk_state.py, ssd_state_passing.py,
 * ssd_bmm.py, ssd_chunk_scan.py).  Per batch b, head h (group g = h / (nheads / ngroups)):
 *
 *   dt_t   = clamp(softplus(dt_t + dt_bias_h) | dt_t + dt_bias_h, dt_min, dt_max)
 *   h_t    = exp(A_h dt_t) h_{t-1} + dt_t x_t B_t^T            ([headdim, dstate])
 *   y_t    = h_t C_t + D x_t ;  out_t = y_t * silu(z_t)
 *
 * with h_{-1} = initial_states (or 0) and the state reset where seq_idx changes, computed
 * in chunks of chunk_size steps as the reference does: per-chunk cumulative decay, chunk
 * states, state passing across chunks, C B^T within chunks, and the chunk scan.
 *
 * Conventions
 *   x, z, out, out_x     : [batch, seqlen, nheads, headdim], io_dtype, headdim stride 1
 *   dt                   : [batch, seqlen, nheads], io_dtype, any strides
 *   A                    : [nheads] fp32;  dt_bias: [nheads] fp32 (optional)
 *   B, C                 : [batch, seqlen, ngroups, dstate], io_dtype, dstate stride 1
 *   D                    : [nheads] or [nheads, headdim] fp32 (optional)
 *   initial_states       : [batch, nheads, headdim, dstate] fp32, any strides (optional)
 *   seq_idx              : [batch, seqlen] int32, any strides (optional)
 *   final_states         : [batch, nheads, headdim, dstate] fp32 contiguous (optional out)
 * Supported: headdim 1..128, dstate 1..256, chunk_size 64, 128, 192 or 256, io_dtype bf16,
 * fp16 or fp32.  The kernels' tiles are headdim 32 / 64 / 128 and dstate 32 / 64 / 128 / 256;
 * other sizes run on the next tile size up, through zero-padded workspace copies of x, z,
 * dout (headdim) and B, C (dstate) and padded out, out_x, dx, dz copied back (the workspace
 * sizes include them).  Rows accessed with 16-byte vector loads and stores need a unit last
 * stride and must start on 16-byte boundaries: x, z, out, out_x, dout, dx at a tile headdim,
 * B and C at a tile dstate.  Errors and streams as in s6scan.h.
 */
#ifndef S6_SSD_H
#define S6_SSD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct S6SsdProblem {
  int64_t batch, seqlen, nheads, headdim, ngroups, dstate, chunk_size;
  int32_t io_dtype;        /* s6_dtype of x, z, B, C, dt, out */
  int32_t has_D, D_has_hdim, has_z, has_dt_bias, dt_softplus;
  int32_t has_initial_states, has_seq_idx;
  float dt_min, dt_max;    /* dt_limit; (0, +inf) = none */
} S6SsdProblem;

typedef struct S6SsdFwdArgs {
  S6SsdProblem p;
  const void* x;               int64_t x_stride[4];
  const void* dt;              int64_t dt_stride[3];
  const float* A;              int64_t A_stride;
  const void* B;               int64_t B_stride[4];
  const void* C;               int64_t C_stride[4];
  const float* D;              int64_t D_stride[2];
  const void* z;               int64_t z_stride[4];
  const float* dt_bias;        int64_t dt_bias_stride;
  const float* initial_states; int64_t initial_states_stride[4];
  const int32_t* seq_idx;      int64_t seq_idx_stride[2];
  void* out;                   int64_t out_stride[4];
  void* out_x;                 int64_t out_x_stride[4];   /* y before the z gate; NULL = not written */
  float* final_states;         /* NULL = not written */
  void* workspace;             size_t workspace_bytes;
  /* Optional hipEvent_t pair (NULL = off), recorded on the call's stream right before and
   * after the chunk-scan kernel, so a caller can time that kernel alone.  No counterpart in
   * the reference; it exists for roofline measurement. */
  void* kernel_events[2];
  /* Optional per-sequence final states (return_varlen_states; replaces chunk_state_varlen,
   * ssd_chunk_state.py:884-910): with batch == 1 and cu_seqlens [nseq + 1] int32 (device) the
   * state at the end of each sequence cu_seqlens[i] .. cu_seqlens[i + 1] - 1 is written to
   * varlen_states [nseq, nheads, headdim, dstate] contiguous, io_dtype.  The carried part
   * comes from the passed states, so seq_idx should mark the same boundaries.  Sequences
   * whose bounds are not 0 <= start < end <= seqlen get a zero state.  NULL = off. */
  const int32_t* cu_seqlens;   int64_t nseq;
  void* varlen_states;
} S6SsdFwdArgs;

typedef struct S6SsdBwdArgs {
  S6SsdProblem p;
  const void* x;               int64_t x_stride[4];
  const void* dt;              int64_t dt_stride[3];
  const float* A;              int64_t A_stride;
  const void* B;               int64_t B_stride[4];
  const void* C;               int64_t C_stride[4];
  const float* D;              int64_t D_stride[2];
  const void* z;               int64_t z_stride[4];
  const float* dt_bias;        int64_t dt_bias_stride;
  const float* initial_states; int64_t initial_states_stride[4];
  const int32_t* seq_idx;      int64_t seq_idx_stride[2];
  const void* dout;            int64_t dout_stride[4];   /* headdim stride 1, 16-byte rows */
  const void* out_x;           int64_t out_x_stride[4];  /* forward y before the z gate; has_z */
  const float* dfinal_states;  int64_t dfinal_states_stride[4];  /* NULL = zero */
  void* dx;                    int64_t dx_stride[4];
  void* ddt;                   int64_t ddt_stride[3];
  float* dA;                   /* [nheads] */
  void* dB;                    int64_t dB_stride[4];
  void* dC;                    int64_t dC_stride[4];
  float* dD;                   /* [nheads] or [nheads, headdim] contiguous; has_D */
  void* dz;                    int64_t dz_stride[4];     /* has_z */
  float* ddt_bias;             /* [nheads]; has_dt_bias */
  float* dinitial_states;      /* [batch, nheads, headdim, dstate] contiguous; NULL = not written */
  void* workspace;             size_t workspace_bytes;
} S6SsdBwdArgs;

int s6_ssd_validate_fwd(const S6SsdFwdArgs* a);
size_t s6_ssd_fwd_workspace_bytes(const S6SsdProblem* p);

/* Replaces _mamba_chunk_scan_combined_fwd (ssd_combined.py:281-332). */
int s6_ssd_fwd(const S6SsdFwdArgs* a, void* stream);

int s6_ssd_validate_bwd(const S6SsdBwdArgs* a);
size_t s6_ssd_bwd_workspace_bytes(const S6SsdProblem* p);

/* Replaces _mamba_chunk_scan_combined_bwd (ssd_combined.py:335-452): writes dx, ddt, dA, dB,
 * dC and, when present, dD, dz, ddt_bias, dinitial_states (overwritten, deterministic). */
int s6_ssd_bwd(const S6SsdBwdArgs* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* S6_SSD_H */
