/*
 * s6scan -- MI355X (gfx950) S6 selective scan, C ABI.
 *
 * This is the native boundary below the reference's Python autograd op
 * ``SelectiveScanFn`` (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/
 * selective_scan_interface.py:19-88).  The reference binds an un-vendored pybind module
 * ``selective_scan_cuda`` with
 *     fwd(u, delta, A, B, C, D, z, delta_bias, delta_softplus) -> (out, x, [out_z])
 *         (selective_scan_interface.py:42, 225-227)
 *     bwd(u, delta, A, B, C, D, z, delta_bias, dout, x, out, dz, delta_softplus,
 *         recompute_out_z) -> (du, ddelta, dA, dB, dC, dD, ddelta_bias, [dz, [out_z]])
 *         (selective_scan_interface.py:67-70, 263-267)
 * s6_fwd / s6_bwd replace those two calls.  The arguments carry the same tensors as
 * plain device pointers plus element strides; the caller allocates every tensor
 * (outputs and workspace included) and the library never allocates device memory.
 *
 * Conventions
 *   u, delta, z, out, out_z, dout, du, ddelta, dz : [batch, dim, seqlen], any strides
 *   A                                              : [dim, dstate] fp32, any strides
 *   B, C, dB, dC                                   : [batch, ngroups, dstate, seqlen], any strides
 *   D, delta_bias, dD, ddelta_bias                 : [dim] fp32, any stride
 *   x_ckpt                                         : [batch, s6_num_checkpoints(), dim, dstate]
 *                                                    fp32, contiguous unless x_ckpt_stride
 *                                                    says otherwise (element strides of the
 *                                                    four axes, the dstate one 1; all zero =
 *                                                    contiguous); entry k is the state after
 *                                                    step min((k+1)*S6_CKPT_INTERVAL,
 *                                                    seqlen)-1, so x_ckpt[:, -1] is the final
 *                                                    state.  s6_bwd never reads that last
 *                                                    entry.  It plays the role of the
 *                                                    reference kernel's saved `x`
 *                                                    (selective_scan_interface.py:42-47).
 *   last_state                                     : [batch, dim, dstate] fp32 contiguous
 *                                                    ([nseq, dim, dstate] for varlen)
 *   Varlen (nseq > 0): batch == 1, cu_seqlens is a device int32 [nseq+1] with
 *   cu_seqlens[0] == 0, non-decreasing, cu_seqlens[nseq] == seqlen; the state is reset to
 *   zero at every sequence start (the seq_idx convention of the reference's chunked scans,
 *   ssd_state_passing.py:76-78).
 *
 * Errors: every entry point returns S6_OK (0) or a negative S6_E* code; the message of the
 * last failure on the calling thread is returned by s6_last_error().
 * Streams: all device work is enqueued on the given hipStream_t (NULL = default stream),
 * asynchronously; the library keeps no pointers after return and, apart from the scratch
 * array of s6_fwd_noalloc, holds no global device state, so calls on different streams
 * with different workspaces may overlap.
 */
#ifndef S6SCAN_H
#define S6SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S6_ABI_VERSION 6
#define S6_CKPT_INTERVAL 8    /* steps between saved states in x_ckpt */
#define S6_MAX_DSTATE_FWD 64
#define S6_MAX_DSTATE_BWD 64
#define S6_NOALLOC_SCRATCH_BYTES 67108864  /* scratch of s6_fwd_noalloc, per device (64 MiB) */

enum s6_dtype { S6_F32 = 0, S6_BF16 = 1, S6_F16 = 2 };

enum s6_status {
  S6_OK = 0,
  S6_E_INVALID = -1,      /* bad argument: shape, stride, dtype, null pointer */
  S6_E_UNSUPPORTED = -2,  /* valid in the reference but not provided by this library */
  S6_E_WORKSPACE = -3,    /* workspace missing or too small */
  S6_E_HIP = -4           /* a HIP runtime call failed */
};

typedef struct S6Problem {
  int64_t batch, dim, seqlen, dstate, ngroups;
  int32_t io_dtype;        /* u, delta, z, out, out_z, dout, du, ddelta, dz */
  int32_t bc_dtype;        /* B, C (dB, dC are always fp32) */
  int32_t has_D, has_z, has_delta_bias, delta_softplus;
  int32_t nseq;            /* 0: dense batch; > 0: packed varlen, batch must be 1 */
} S6Problem;

typedef struct S6FwdArgs {
  S6Problem p;
  const void* u;            int64_t u_stride[3];
  const void* delta;        int64_t delta_stride[3];
  const float* A;           int64_t A_stride[2];
  const void* B;            int64_t B_stride[4];
  const void* C;            int64_t C_stride[4];
  const float* D;           int64_t D_stride;
  const void* z;            int64_t z_stride[3];
  const float* delta_bias;  int64_t delta_bias_stride;
  const int32_t* cu_seqlens;
  void* out;                int64_t out_stride[3];    /* y + D*u (before the z gate)     */
  void* out_z;              int64_t out_z_stride[3];  /* out * silu(z); has_z only       */
  float* x_ckpt;            /* may be NULL (no backward will follow)                    */
  int64_t x_ckpt_stride[4]; /* [batch, checkpoint, dim, dstate]: [3] == 1, or all zero =
                             * contiguous                                                 */
  float* last_state;        /* may be NULL                                               */
  void* workspace;          size_t workspace_bytes;
  /* Optional hipEvent_t pair (NULL = off), recorded on the call's stream right before and
   * after the main scan kernel, so a caller can time that kernel alone.  No counterpart in
   * the reference; it exists for roofline measurement. */
  void* kernel_events[2];
} S6FwdArgs;

typedef struct S6BwdArgs {
  S6Problem p;
  const void* u;            int64_t u_stride[3];
  const void* delta;        int64_t delta_stride[3];
  const float* A;           int64_t A_stride[2];
  const void* B;            int64_t B_stride[4];
  const void* C;            int64_t C_stride[4];
  const float* D;           int64_t D_stride;
  const void* z;            int64_t z_stride[3];
  const float* delta_bias;  int64_t delta_bias_stride;
  const int32_t* cu_seqlens;
  const void* dout;         int64_t dout_stride[3];
  const float* x_ckpt;      /* as written by s6_fwd for the same inputs                  */
  int64_t x_ckpt_stride[4]; /* as passed to s6_fwd                                       */
  const void* out;          int64_t out_stride[3];    /* pre-gate output; has_z only    */
  void* du;                 int64_t du_stride[3];
  void* ddelta;             int64_t ddelta_stride[3];
  float* dA;                int64_t dA_stride[2];
  float* dB;                int64_t dB_stride[4];
  float* dC;                int64_t dC_stride[4];
  float* dD;                int64_t dD_stride;        /* has_D only                     */
  void* dz;                 int64_t dz_stride[3];     /* has_z only                     */
  /* Optional (NULL = not written; has_z only): out * silu(z) recomputed from out and z, the
   * reference's recompute_out_z (selective_scan_interface.py:263-267). */
  void* out_z;              int64_t out_z_stride[3];
  float* ddelta_bias;       int64_t ddelta_bias_stride; /* has_delta_bias only          */
  void* workspace;          size_t workspace_bytes;
  void* kernel_events[2];   /* as in S6FwdArgs, around the main backward kernel          */
} S6BwdArgs;

/* ABI version of the loaded library (S6_ABI_VERSION it was built with). */
int s6_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* s6_last_error(void);

/* Host-only shape/dtype check of a problem (no device access). */
int s6_validate_problem(const S6Problem* p);

/* Host-only check of forward / backward arguments (shapes, strides, null pointers,
 * workspace size).  s6_fwd / s6_bwd run the same checks before launching. */
int s6_validate_fwd(const S6FwdArgs* a);
int s6_validate_bwd(const S6BwdArgs* a);

/* Host-only check of packed-varlen offsets held in HOST memory (a copy of the device
 * vector passed as cu_seqlens): nseq >= 1, cu[0] == 0, non-decreasing, cu[nseq] == seqlen.
 * Returns S6_E_INVALID with a message naming the first violation.  s6_fwd / s6_bwd cannot
 * read device memory before launching, so a caller passing device offsets it has not
 * checked this way gets unspecified results for a malformed vector (the kernels still keep
 * every store inside the output tensors).  Same convention as the reference's varlen
 * chunked scan (ssd_combined.py:576-577, ssd_state_passing.py:76-78). */
int s6_validate_cu_seqlens(const int32_t* cu_host, int64_t nseq, int64_t seqlen);

/* Host-only: 1 if s6_fwd runs this problem on the single-pass kernel (one lane per
 * (channel, state)), 0 if on the chunked kernels (chunk summaries, carry, output pass), or a
 * negative code for an invalid problem.  From the problem alone: arguments with L-contiguous
 * u / delta / out (z / out_z) can also take the single-pass kernel (s6_fwd_kernel).  Follows the environment override S6_FWD_PATH=lanes /
 * chunked as s6_fwd does.  No counterpart in the reference: it names the kernel a caller is
 * timing or profiling. */
int s6_fwd_single_pass(const S6Problem* p);

/* Host-only: which forward kernels s6_fwd runs for these arguments, or a negative code for
 * invalid arguments (the workspace is not checked):
 *   S6_FWD_SINGLE_PASS   the single-pass kernel (as s6_fwd_single_pass says from the problem
 *                        alone; arguments whose u / delta / out (z / out_z) have a contiguous
 *                        time axis also take it with the z gate and at any wave count);
 *   S6_FWD_CHUNKED_ROWS  the chunked kernels moving u / delta / z / out / out_z in whole
 *                        8-step row blocks per lane (those tensors L-contiguous with 16-byte
 *                        aligned rows and blocks, seqlen a multiple of 8, dstate <= 32);
 *   S6_FWD_CHUNKED       the chunked kernels, one step at a time (any strides).
 * Follows the environment overrides S6_FWD_PATH=lanes / chunked and S6_FWD_ROWVEC=0 (per-step
 * accesses) as s6_fwd does; the two chunked forms give bit-identical results.  No
 * counterpart in the reference: it names the kernels a caller is timing. */
#define S6_FWD_CHUNKED 0
#define S6_FWD_CHUNKED_ROWS 1
#define S6_FWD_SINGLE_PASS 2
int s6_fwd_kernel(const S6FwdArgs* a);

/* Host-only: 1 if s6_bwd moves u, delta, dout, du, ddelta (with z: z, out, dz and out_z when
 * given) in whole 8-step row blocks per lane (each L-contiguous with 16-byte aligned rows and
 * blocks, seqlen a multiple of 8, dstate <= 16), 0 if one step at a time, or a negative code
 * for an invalid problem (the other arguments are not checked).  Override S6_BWD_ROWVEC=0;
 * both forms give bit-identical results.  No counterpart in the reference. */
int s6_bwd_row_blocks(const S6BwdArgs* a);

/* Number of x_ckpt entries along the sequence: ceil(seqlen / S6_CKPT_INTERVAL). */
int64_t s6_num_checkpoints(const S6Problem* p);

/* Device workspace the calls need, in bytes (0 is possible). */
size_t s6_fwd_workspace_bytes(const S6Problem* p);
size_t s6_bwd_workspace_bytes(const S6Problem* p);

/* Forward scan: replaces selective_scan_cuda.fwd (selective_scan_interface.py:42). */
int s6_fwd(const S6FwdArgs* a, void* stream);

/* Forward scan that allocates nothing.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as s6_fwd, except
 * that a->workspace / a->workspace_bytes are ignored: the workspace is a library-owned
 * array of S6_NOALLOC_SCRATCH_BYTES on each device, kept until the process ends.  A problem
 * whose workspace (s6_fwd_workspace_bytes) exceeds that returns S6_E_WORKSPACE before any
 * device work.  The caller still allocates every input and output.  All calls on one
 * device share its array: calls that overlap in time on one device (different streams, or
 * threads) race and must be serialised by the caller.  Calls no hipMalloc / hipFree. */
int s6_fwd_noalloc(const S6FwdArgs* a, void* stream);

/* Backward scan: replaces selective_scan_cuda.bwd (selective_scan_interface.py:67-70).
 * dA, dB, dC, dD, ddelta_bias are overwritten (not accumulated into). */
int s6_bwd(const S6BwdArgs* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* S6SCAN_H */
