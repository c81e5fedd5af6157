"""CPU restatement of the fused Mamba block and its causal conv1d -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and the other checker legs named in ``oracle/selective_scan_ref.py``)
may import this module, as the checker of ``s6scan.causal_conv1d`` and
``s6scan.mamba_inner``.

``causal_conv1d_ref`` is the reference's own non-CUDA convolution,
``act(conv1d(x)[..., :seqlen])`` with ``nn.Conv1d(groups=dim, padding=width - 1)``
(/root/reference/zoology/zoology/mixers/mamba.py:55-62, 159-161), written with the
functional ``F.conv1d`` on a ``[dim, width]`` weight (the ``"d 1 w -> d w"`` layout of
mamba.py:165 and selective_scan_interface.py:185).

``causal_conv1d_loop64`` is a float64 NumPy loop of the defining sum
``out[b, d, t] = act(bias[d] + sum_k w[d, k] x[b, d, t - W + 1 + k])`` (x = 0 before t = 0),
independent of torch's convolution; tests pin ``causal_conv1d_ref`` with it, with the
impulse response (a unit impulse at s gives out[s + j] = w[W - 1 - j] + bias) and with the
width-2 identity (w = [0, 1]).

``mamba_inner_ref`` restates ``mamba_inner_ref`` (selective_scan_interface.py:310-356) op
for op: conv + SiLU on the x half of xz, ``x_dbl = F.linear(conv, x_proj_weight)``,
``delta = delta_proj_weight @ x_dbl[:, :dt_rank].T``, B / C from ``x_dbl`` (plus their
optional biases), the selective scan with z, D, delta_bias and softplus
(``selective_scan_ref``), and ``F.linear(y, out_proj_weight, out_proj_bias)``.  Gradients
are autograd through it (the reference's ``MambaInnerFn.backward`` computes the same
derivatives by hand).  Pinned in ``tests/test_oracle_mamba_inner.py`` against a float64 composition
of the two brute forces (``causal_conv1d_loop64`` and ``brute64.scan_fwd64``).
"""
import numpy as np
import torch
import torch.nn.functional as F

from .selective_scan_ref import selective_scan_ref


def causal_conv1d_ref(x, weight, bias=None, activation=None):
    """x: [batch, dim, seqlen]; weight: [dim, width]; bias: [dim] or None; activation None,
    "silu" or "swish".  Computes in x's dtype (callers pass fp32 / fp64)."""
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    dim, width = weight.shape
    seqlen = x.shape[-1]
    out = F.conv1d(x, weight.unsqueeze(1).to(x.dtype),
                   bias.to(x.dtype) if bias is not None else None,
                   padding=width - 1, groups=dim)[..., :seqlen]
    return F.silu(out) if activation in ("silu", "swish") else out


def causal_conv1d_loop64(x, weight, bias=None, silu=False):
    """Float64 loop over the defining sum; numpy arrays in, numpy array out."""
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    batch, dim, seqlen = x.shape
    width = w.shape[1]
    out = np.zeros_like(x)
    for b in range(batch):
        for d in range(dim):
            for t in range(seqlen):
                acc = 0.0 if bias is None else float(bias[d])
                for k in range(width):
                    s = t - width + 1 + k
                    if s >= 0:
                        acc += w[d, k] * x[b, d, s]
                out[b, d, t] = acc / (1.0 + np.exp(-acc)) if silu else acc
    return out


def mamba_inner_ref(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                    out_proj_weight, out_proj_bias, A, B=None, C=None, D=None,
                    delta_bias=None, B_proj_bias=None, C_proj_bias=None, delta_softplus=True,
                    compute_dtype=torch.float32):
    """xz: (batch, 2 * d_inner, seqlen); conv1d_weight: (d_inner, 1, width) or
    (d_inner, width).  Returns (batch, seqlen, d_model).  ``compute_dtype`` is the scan's
    internal precision (fp32 as the reference kernel; float64 for the pinning tests)."""
    L = xz.shape[-1]
    delta_rank = delta_proj_weight.shape[1]
    d_state = A.shape[-1]
    x, z = xz.chunk(2, dim=1)
    w = conv1d_weight.flatten(1) if conv1d_weight.dim() == 3 else conv1d_weight
    x = causal_conv1d_ref(x, w, conv1d_bias, activation="silu")
    x_dbl = F.linear(x.transpose(1, 2).reshape(-1, x.shape[1]), x_proj_weight)  # (bl, d)
    delta = delta_proj_weight @ x_dbl[:, :delta_rank].t()
    delta = delta.reshape(delta.shape[0], -1, L).transpose(0, 1)  # "d (b l) -> b d l"
    if B is None:
        B = x_dbl[:, delta_rank:delta_rank + d_state]
        if B_proj_bias is not None:
            B = B + B_proj_bias.to(dtype=B.dtype)
        B = B.reshape(-1, L, d_state).transpose(1, 2).contiguous()  # "(b l) n -> b n l"
    if C is None:
        C = x_dbl[:, -d_state:]
        if C_proj_bias is not None:
            C = C + C_proj_bias.to(dtype=C.dtype)
        C = C.reshape(-1, L, d_state).transpose(1, 2).contiguous()
    y = selective_scan_ref(x, delta, A, B, C, D, z=z, delta_bias=delta_bias,
                           delta_softplus=delta_softplus, compute_dtype=compute_dtype)
    return F.linear(y.transpose(1, 2), out_proj_weight, out_proj_bias)
