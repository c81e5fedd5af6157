"""One recurrent decode step of the S6 state on the gfx950 kernel of ``libs6scan.so``.

Same signature, shapes, in-place state update and return value as the reference's
``selective_state_update`` (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/
selective_state_update.py:121-201; semantics ``selective_state_update_ref`` :204-265):

    selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False) -> out

* state: (batch, dim, dstate) or (batch, nheads, dim, dstate), updated in place, any
  strides (e.g. a slice of a larger inference cache), fp32 / bf16 / fp16;
* x, dt, z: (batch, dim) or (batch, nheads, dim); A: (dim, dstate) or (nheads, dim,
  dstate); B, C: (batch, dstate) or (batch, ngroups, dstate); D, dt_bias: (dim,) or
  (nheads, dim).  Zero strides on A and dt (the reference's tied-head-dim form, one value
  per head) are read as given.
* out has x's shape and dtype.

All arithmetic is fp32 in the kernel; ``out`` uses the updated fp32 state before it is
rounded to the state's dtype, as the reference kernel does.  There is no CPU path.
"""
import ctypes

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _st(t, n):
    return tuple(t.stride()) if t is not None else (0,) * n


# Rank of each argument without a head axis, and where the head (or group) axis of size 1
# goes when it is absent: the reference accepts both forms of every argument.
_HEADLESS = {"state": (3, 1), "x": (2, 1), "dt": (2, 1), "A": (2, 0), "B": (2, 1), "C": (2, 1),
             "D": (1, 0), "z": (2, 1), "dt_bias": (1, 0)}


def _with_heads(name, t):
    if t is None:
        return None
    rank, axis = _HEADLESS[name]
    return t.unsqueeze(axis) if t.dim() == rank else t


def _require(ok, what):
    # shape errors are AssertionErrors, as in the reference wrapper
    if not ok:
        raise AssertionError(f"selective_state_update: {what}")


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False):
    has_heads = state.dim() > 3
    state, x, dt, A, B, C, D, z, dt_bias = (
        _with_heads(n, t) for n, t in zip(("state", "x", "dt", "A", "B", "C", "D", "z", "dt_bias"),
                                          (state, x, dt, A, B, C, D, z, dt_bias)))
    batch, nheads, dim, dstate = state.shape
    ngroups = B.shape[1]
    want = {"x": (batch, nheads, dim), "dt": (batch, nheads, dim), "z": (batch, nheads, dim),
            "A": (nheads, dim, dstate), "B": (batch, ngroups, dstate),
            "C": (batch, ngroups, dstate), "D": (nheads, dim), "dt_bias": (nheads, dim)}
    for name, t in (("x", x), ("dt", dt), ("A", A), ("B", B), ("C", C), ("D", D), ("z", z),
                    ("dt_bias", dt_bias)):
        if t is not None:
            _require(tuple(t.shape) == want[name],
                     f"{name} has shape {tuple(t.shape)}, expected {want[name]}")
    _require(nheads % ngroups == 0, "nheads must be divisible by ngroups")
    if not state.is_cuda:
        raise RuntimeError("selective_state_update: tensors must be on a ROCm device (no CPU path)")
    for t, name in ((state, "state"), (x, "x"), (B, "B")):
        if t.dtype not in _DTYPES:
            raise TypeError(f"selective_state_update: unsupported {name} dtype {t.dtype}")
    if dt.dtype != x.dtype:
        dt = dt.to(x.dtype)
    if z is not None and z.dtype != x.dtype:
        z = z.to(x.dtype)
    if C.dtype != B.dtype:
        C = C.to(B.dtype)
    f32 = lambda t: t if t is None or t.dtype == torch.float32 else t.float()
    A, D, dt_bias = f32(A), f32(D), f32(dt_bias)
    with torch.cuda.device(x.device):
        out = torch.empty_like(x)
        a = _lib.S6StateUpdateArgs()
        a.batch, a.nheads, a.dim, a.dstate, a.ngroups = batch, nheads, dim, dstate, ngroups
        a.state_dtype, a.io_dtype, a.bc_dtype = _DTYPES[state.dtype], _DTYPES[x.dtype], _DTYPES[B.dtype]
        a.has_D, a.has_z, a.has_dt_bias = int(D is not None), int(z is not None), int(dt_bias is not None)
        a.dt_softplus = int(bool(dt_softplus))
        a.state, a.state_stride = _ptr(state), _st(state, 4)
        a.x, a.x_stride = _ptr(x), _st(x, 3)
        a.dt, a.dt_stride = _ptr(dt), _st(dt, 3)
        a.dt_bias, a.dt_bias_stride = _ptr(dt_bias), _st(dt_bias, 2)
        a.A, a.A_stride = _ptr(A), _st(A, 3)
        a.B, a.B_stride = _ptr(B), _st(B, 3)
        a.C, a.C_stride = _ptr(C), _st(C, 3)
        a.D, a.D_stride = _ptr(D), _st(D, 2)
        a.z, a.z_stride = _ptr(z), _st(z, 3)
        a.out, a.out_stride = _ptr(out), _st(out, 3)
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check(_lib.LIB.s6_selective_state_update(ctypes.byref(a), ctypes.c_void_p(stream)),
                   "s6_selective_state_update")
    if not has_heads:
        out = out.squeeze(1)
    return out
