/*
 * s6scan selective_state_update -- MI355X (gfx950), C ABI.
 *
 * One recurrent decode step of the S6 state: replaces the Triton kernel behind
 * `selective_state_update` (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/
 * selective_state_update.py:18-118, wrapper :121-201; reference semantics
 * `selective_state_update_ref` :204-265).  For every (b, h, d):
 *
 *     dt    = softplus(dt[b,h,d] + dt_bias[h,d])            (softplus optional, threshold 20)
 *     state = state * exp(A[h,d,:] * dt) + (B[b,g,:] * dt) * x[b,h,d]   (updated in place)
 *     out   = sum_n state[n] * C[b,g,n] + D[h,d] * x[b,h,d]
 *     out  *= silu(z[b,h,d])                                 (if z is given)
 *
 * with g = h / (nheads / ngroups), all arithmetic in fp32 and `out` taken from the fp32
 * state before it is rounded to the state's storage type.
 *
 * Conventions
 *   state          : [batch, nheads, dim, dstate], state_dtype, any strides (updated in place)
 *   x, dt, z, out  : [batch, nheads, dim], io_dtype, any strides
 *   A              : [nheads, dim, dstate] fp32, any strides (zero strides express the
 *                    reference's tied-head-dim case: one A per head)
 *   B, C           : [batch, ngroups, dstate], bc_dtype, any strides
 *   D, dt_bias     : [nheads, dim] fp32, any strides (NULL when absent)
 * Errors and streams as in s6scan.h (S6_OK or a negative S6_E* code, s6_last_error(),
 * stream-ordered, no device allocation, no pointers kept after return).  No workspace.
 */
#ifndef S6_SELECTIVE_STATE_UPDATE_H
#define S6_SELECTIVE_STATE_UPDATE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S6_SSU_MAX_DSTATE 256

typedef struct S6StateUpdateArgs {
  int64_t batch, nheads, dim, dstate, ngroups;
  int32_t state_dtype, io_dtype, bc_dtype;   /* s6_dtype values */
  int32_t has_D, has_z, has_dt_bias, dt_softplus;
  void* state;          int64_t state_stride[4];
  const void* x;        int64_t x_stride[3];
  const void* dt;       int64_t dt_stride[3];
  const float* dt_bias; int64_t dt_bias_stride[2];
  const float* A;       int64_t A_stride[3];
  const void* B;        int64_t B_stride[3];
  const void* C;        int64_t C_stride[3];
  const float* D;       int64_t D_stride[2];
  const void* z;        int64_t z_stride[3];
  void* out;            int64_t out_stride[3];
} S6StateUpdateArgs;

/* Host-only check (no device access); s6_selective_state_update runs it first. */
int s6_validate_state_update(const S6StateUpdateArgs* a);

/* Replaces selective_state_update (selective_state_update.py:121-201). */
int s6_selective_state_update(const S6StateUpdateArgs* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* S6_SELECTIVE_STATE_UPDATE_H */
