"""Causal depthwise conv1d on the gfx950 kernels of ``libs6scan.so``.

Replaces the ``causal_conv1d`` package that the reference's Mamba paths import
(/root/reference/zoology/zoology/mixers/mamba_ssm/ops/selective_scan_interface.py:9-14,
187-189, 299-301; zoology/mixers/mamba.py:12, 163-169):

* ``causal_conv1d_fwd(x, weight, bias, seq_idx, initial_states, final_states_out,
  silu_activation) -> out`` and ``causal_conv1d_bwd(x, weight, bias, dout, seq_idx,
  initial_states, dfinal_states, dx, return_dinitial_states, silu_activation) -> (dx,
  dweight, dbias, None)``: the native-module calls ``MambaInnerFn`` makes;
* ``causal_conv1d_fn(x, weight, bias=None, seq_idx=None, activation=None)``: the
  differentiable function (positional order of the call at mamba.py:163-169).

``out[b, d, t] = act(bias[d] + sum_k weight[d, k] x[b, d, t - width + 1 + k])``, x taken as
zero before t = 0, width 2..4, act = identity or SiLU.  x: [batch, dim, seqlen] in fp32,
bf16 or fp16 with any strides; channel-last storage (``x.stride(1) == 1``) takes the
vectorised kernel, and out / dx follow x's layout.  weight [dim, width] and bias [dim] may
have any float dtype (the kernels read fp32 copies); dweight / dbias come back in their
dtypes.  ``seq_idx``, ``initial_states`` and final states, which the reference's S6 paths
never pass, raise ``NotImplementedError``.
"""
import ctypes

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _check(x, weight, bias):
    if x.dim() != 3:
        raise ValueError("causal_conv1d: x must be [batch, dim, seqlen]")
    if not x.is_cuda:
        raise RuntimeError("causal_conv1d: x must be on a ROCm device (no CPU path)")
    if x.dtype not in _DTYPES:
        raise TypeError(f"causal_conv1d: unsupported dtype {x.dtype}")
    if weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError("causal_conv1d: weight must be [dim, width]")
    if not 2 <= weight.shape[1] <= 4:
        raise NotImplementedError("causal_conv1d: width must be between 2 and 4")
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != x.shape[1]):
        raise ValueError("causal_conv1d: bias must be [dim]")
    for t in (weight, bias):
        if t is not None and t.device != x.device:
            raise ValueError("causal_conv1d: all tensors must be on one device")


def _new_like(x):
    """Empty tensor of x's shape and dtype, channel-last when x's channels are contiguous
    (x may be a strided view such as one half of a channel-last xz buffer)."""
    if x.stride(1) == 1 and x.shape[1] > 1:
        b, d, l = x.shape
        return torch.empty(b, l, d, dtype=x.dtype, device=x.device).mT
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _unsupported(seq_idx, initial_states, final_states):
    if seq_idx is not None or initial_states is not None or final_states is not None:
        raise NotImplementedError(
            "causal_conv1d: seq_idx / initial_states / final_states are not supported")


def _problem(x, weight, silu):
    batch, dim, seqlen = x.shape
    return _lib.S6ConvProblem(batch, dim, seqlen, weight.shape[1], _DTYPES[x.dtype],
                              int(bool(silu)))


def causal_conv1d_fwd(x, weight, bias, seq_idx=None, initial_states=None,
                      final_states_out=None, silu_activation=False):
    """Forward of the native module (selective_scan_interface.py:187-189)."""
    _check(x, weight, bias)
    _unsupported(seq_idx, initial_states, final_states_out)
    w32 = weight.float()
    b32 = bias.float() if bias is not None else None
    with torch.cuda.device(x.device):
        out = _new_like(x)
        a = _lib.S6ConvFwdArgs()
        a.p = _problem(x, weight, silu_activation)
        a.x, a.x_stride = _ptr(x), tuple(x.stride())
        a.weight, a.weight_stride = _ptr(w32), tuple(w32.stride())
        a.bias, a.bias_stride = _ptr(b32), (b32.stride(0) if b32 is not None else 0)
        a.out, a.out_stride = _ptr(out), tuple(out.stride())
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check(_lib.LIB.s6_causal_conv1d_fwd(ctypes.byref(a), ctypes.c_void_p(stream)),
                   "s6_causal_conv1d_fwd")
    return out


def causal_conv1d_bwd(x, weight, bias, dout, seq_idx=None, initial_states=None,
                      dfinal_states=None, dx=None, return_dinitial_states=False,
                      silu_activation=False):
    """Backward of the native module (selective_scan_interface.py:299-301).  Returns
    ``(dx, dweight, dbias, None)``; dbias is None without bias.  ``dx``: optional
    preallocated output of x's shape and dtype (any strides)."""
    _check(x, weight, bias)
    _unsupported(seq_idx, initial_states, dfinal_states)
    if return_dinitial_states:
        raise NotImplementedError("causal_conv1d: initial-state gradients are not supported")
    if dout.shape != x.shape:
        raise ValueError("causal_conv1d: dout must have x's shape")
    if dout.dtype != x.dtype:
        dout = dout.to(x.dtype)
    w32 = weight.float()
    b32 = bias.float() if bias is not None else None
    with torch.cuda.device(x.device):
        if dx is None:
            dx = _new_like(x)
        elif dx.shape != x.shape or dx.dtype != x.dtype or dx.device != x.device:
            raise ValueError("causal_conv1d: dx must match x in shape, dtype and device")
        dw = torch.empty(weight.shape, dtype=torch.float32, device=x.device)
        db = torch.empty(x.shape[1], dtype=torch.float32, device=x.device) if bias is not None else None
        a = _lib.S6ConvBwdArgs()
        a.p = _problem(x, weight, silu_activation)
        a.x, a.x_stride = _ptr(x), tuple(x.stride())
        a.weight, a.weight_stride = _ptr(w32), tuple(w32.stride())
        a.bias, a.bias_stride = _ptr(b32), (b32.stride(0) if b32 is not None else 0)
        a.dout, a.dout_stride = _ptr(dout), tuple(dout.stride())
        a.dx, a.dx_stride = _ptr(dx), tuple(dx.stride())
        a.dweight, a.dweight_stride = _ptr(dw), tuple(dw.stride())
        a.dbias, a.dbias_stride = _ptr(db), (db.stride(0) if db is not None else 0)
        nbytes = _lib.LIB.s6_causal_conv1d_bwd_workspace_bytes(ctypes.byref(a.p))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        a.workspace, a.workspace_bytes = _ptr(ws), nbytes
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check(_lib.LIB.s6_causal_conv1d_bwd(ctypes.byref(a), ctypes.c_void_p(stream)),
                   "s6_causal_conv1d_bwd")
    dweight = dw.to(weight.dtype)
    dbias = db.to(bias.dtype) if bias is not None else None
    return dx, dweight, dbias, None


def _silu_flag(activation):
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    return activation in ("silu", "swish")


class CausalConv1dFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias=None, activation=None):
        silu = _silu_flag(activation)
        ctx.save_for_backward(x, weight, bias)
        ctx.silu = silu
        return causal_conv1d_fwd(x, weight, bias, silu_activation=silu)

    @staticmethod
    def backward(ctx, dout):
        x, weight, bias = ctx.saved_tensors
        dx, dweight, dbias, _ = causal_conv1d_bwd(x, weight, bias, dout,
                                                  silu_activation=ctx.silu)
        return dx, dweight, dbias, None


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, activation=None):
    """x: [batch, dim, seqlen]; weight: [dim, width]; bias: [dim] or None; activation: None,
    "silu" or "swish".  Returns [batch, dim, seqlen] in x's dtype and layout."""
    _unsupported(seq_idx, None, None)
    return CausalConv1dFn.apply(x, weight, bias, activation)
