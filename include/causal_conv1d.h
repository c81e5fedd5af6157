/*
 * s6scan causal depthwise conv1d -- MI355X (gfx950), C ABI.
 *
 * The short causal convolution in front of the S6 scan in the reference's fused Mamba
 * path.  It replaces the two calls of the un-vendored pybind module `causal_conv1d_cuda`
 * made by `MambaInnerFn` (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/
 * selective_scan_interface.py):
 *     causal_conv1d_fwd(x, weight, bias, None, None, None, True) -> out       (:187-189, :252-254)
 *     causal_conv1d_bwd(x, weight, bias, dout, None, None, None, dx, False, True)
 *         -> (dx, dweight, dbias, None)                                       (:299-301)
 * (the three None arguments are seq_idx, initial_states and final_states, which that path
 * never passes and which this library does not take).
 *
 * Semantics (causal_conv1d_fn with activation None or "silu", width 2..4):
 *     out[b, d, t] = act(bias[d] + sum_{k < width} weight[d, k] * x[b, d, t - width + 1 + k])
 * with x taken as zero before t = 0, i.e. nn.Conv1d(groups=dim, padding=width-1) cut to the
 * first seqlen outputs (mamba.py:159-161 of the reference's zoology Mamba).
 *
 * Conventions
 *   x, out, dout, dx : [batch, dim, seqlen], io_dtype, any strides (channel-last storage,
 *                      stride(1) == 1, takes the vectorised path)
 *   weight, dweight  : [dim, width] fp32, any strides
 *   bias, dbias      : [dim] fp32, any stride; bias NULL = no bias, dbias NULL = not written
 * dweight and dbias are overwritten, not accumulated into.  Errors and streams as in
 * s6scan.h (S6_OK or a negative S6_E* code, s6_last_error(), stream-ordered, no device
 * allocation, no pointers kept after return).
 */
#ifndef S6_CAUSAL_CONV1D_H
#define S6_CAUSAL_CONV1D_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S6_CONV_MAX_WIDTH 4

typedef struct S6ConvProblem {
  int64_t batch, dim, seqlen, width;
  int32_t io_dtype;   /* s6_dtype of x, out, dout, dx */
  int32_t silu;       /* 1: activation "silu" / "swish"; 0: none */
} S6ConvProblem;

typedef struct S6ConvFwdArgs {
  S6ConvProblem p;
  const void* x;        int64_t x_stride[3];
  const float* weight;  int64_t weight_stride[2];
  const float* bias;    int64_t bias_stride;
  void* out;            int64_t out_stride[3];
} S6ConvFwdArgs;

typedef struct S6ConvBwdArgs {
  S6ConvProblem p;
  const void* x;        int64_t x_stride[3];
  const float* weight;  int64_t weight_stride[2];
  const float* bias;    int64_t bias_stride;
  const void* dout;     int64_t dout_stride[3];
  void* dx;             int64_t dx_stride[3];
  float* dweight;       int64_t dweight_stride[2];
  float* dbias;         int64_t dbias_stride;
  void* workspace;      size_t workspace_bytes;
} S6ConvBwdArgs;

/* Host-only checks (no device access); the launches run the same checks first. */
int s6_causal_conv1d_validate_fwd(const S6ConvFwdArgs* a);
int s6_causal_conv1d_validate_bwd(const S6ConvBwdArgs* a);

/* Device workspace of the backward (per-block dweight / dbias partials), in bytes. */
size_t s6_causal_conv1d_bwd_workspace_bytes(const S6ConvProblem* p);

/* Replaces causal_conv1d_cuda.causal_conv1d_fwd (selective_scan_interface.py:187-189). */
int s6_causal_conv1d_fwd(const S6ConvFwdArgs* a, void* stream);

/* Replaces causal_conv1d_cuda.causal_conv1d_bwd (selective_scan_interface.py:299-301). */
int s6_causal_conv1d_bwd(const S6ConvBwdArgs* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* S6_CAUSAL_CONV1D_H */
