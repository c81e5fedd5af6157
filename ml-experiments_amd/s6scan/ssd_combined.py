"""Mamba-2 SSD (``mamba_chunk_scan_combined``) on the gfx950 kernels of ``libs6scan.so``.

Same signature, argument meaning and return values as the reference's
``mamba_chunk_scan_combined`` (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/
ssd_combined.py:563-582, forward :281-332):

    mamba_chunk_scan_combined(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                              initial_states=None, seq_idx=None, cu_seqlens=None,
                              dt_softplus=False, dt_limit=(0.0, inf),
                              return_final_states=False, return_varlen_states=False)
        -> out | (out, final_states) | (out, varlen_states) | (out, final_states, varlen_states)

* x, z: (batch, seqlen, nheads, headdim); dt: (batch, seqlen, nheads); A, dt_bias:
  (nheads,); B, C: (batch, seqlen, ngroups, dstate); D: (nheads,) or (nheads, headdim);
  initial_states: (batch, nheads, headdim, dstate); seq_idx: (batch, seqlen) int32.
* out has x's dtype (bf16, fp16 or fp32); final_states is fp32 (batch, nheads, headdim, dstate).
* return_varlen_states (batch 1, cu_seqlens int32 (nseq + 1,)): the state at the end of each
  packed sequence, (nseq, nheads, headdim, dstate) in x's dtype, forward only, as the
  reference's chunk_state_varlen (ssd_chunk_state.py:884-910).

The forward runs five HIP kernels (chunk cumsum, chunk states and C B^T on MFMA, state
passing, the chunk scan on MFMA; ml-experiments_amd/csrc/s6_ssd.hip); the backward recomputes
the chunk quantities and runs ten more (s6_ssd_bwd.hip), deterministic.  Supported
shapes: headdim 1..128, dstate 1..256 (the kernels' tiles are 32 / 64 / 128 and 32 / 64 /
128 / 256; other sizes run on zero-padded copies inside the library), chunk_size 64, 128, 192
or 256.  There is no CPU path.
"""
import ctypes
import math

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _st(t, n):
    return tuple(t.stride()) if t is not None else (0,) * n


_TILES = {"headdim": (32, 64, 128), "dstate": (32, 64, 128, 256)}


def _rows16(t, axis="headdim"):
    """t with unit last stride and 16-byte aligned rows (a contiguous copy otherwise), as
    the reference makes B / C / x contiguous when their last stride is not 1
    (ssd_combined.py:297-304).  Off the kernels' tile sizes the library copies the tensor
    into a zero-padded buffer element by element, at any strides, so t is passed as it is."""
    if t.shape[-1] not in _TILES[axis]:
        return t
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all((s * es) % 16 == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


def _problem(x, B, chunk_size, D, z, dt_bias, initial_states, seq_idx, dt_softplus, dt_limit):
    batch, seqlen, nheads, headdim = x.shape
    _, _, ngroups, dstate = B.shape
    return _lib.S6SsdProblem(batch, seqlen, nheads, headdim, ngroups, dstate, chunk_size,
                             _DTYPES[x.dtype], int(D is not None),
                             int(D is not None and D.dim() == 2), int(z is not None),
                             int(dt_bias is not None), int(bool(dt_softplus)),
                             int(initial_states is not None), int(seq_idx is not None),
                             float(dt_limit[0]), float(dt_limit[1]))


def _prepare(x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx):
    """Shape checks of the reference (ssd_combined.py:283-306) and the kernel operand forms:
    B, C, z, dt in x's dtype; vector-loaded rows contiguous and 16-byte aligned; A, D,
    dt_bias and the initial states fp32; seq_idx int32."""
    batch, seqlen, nheads, headdim = x.shape
    _, _, ngroups, dstate = B.shape
    assert nheads % ngroups == 0
    assert B.shape == (batch, seqlen, ngroups, dstate)
    assert dt.shape == (batch, seqlen, nheads)
    assert A.shape == (nheads,)
    assert C.shape == B.shape
    if z is not None:
        assert z.shape == x.shape
    if D is not None:
        assert D.shape == (nheads, headdim) or D.shape == (nheads,)
    if seq_idx is not None:
        assert seq_idx.shape == (batch, seqlen)
    if initial_states is not None:
        assert initial_states.shape == (batch, nheads, headdim, dstate)
    if not x.is_cuda:
        raise RuntimeError("mamba_chunk_scan_combined: tensors must be on a ROCm device (no CPU path)")
    if x.dtype not in _DTYPES:
        raise NotImplementedError(f"mamba_chunk_scan_combined: dtype {x.dtype} (bf16, fp16 or fp32 only)")
    dtype = x.dtype
    x, B, C = _rows16(x), _rows16(B.to(dtype), "dstate"), _rows16(C.to(dtype), "dstate")
    if z is not None:
        z = _rows16(z.to(dtype))
    f32 = lambda t: None if t is None else t.float()
    if seq_idx is not None:
        seq_idx = seq_idx.to(torch.int32)
    return (x, dt.to(dtype), f32(A), B, C, f32(D), z, f32(dt_bias), f32(initial_states),
            seq_idx)


def _fill_inputs(a, x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx):
    a.x, a.x_stride = _ptr(x), _st(x, 4)
    a.dt, a.dt_stride = _ptr(dt), _st(dt, 3)
    a.A, a.A_stride = _ptr(A), A.stride(0)
    a.B, a.B_stride = _ptr(B), _st(B, 4)
    a.C, a.C_stride = _ptr(C), _st(C, 4)
    Dm = None if D is None else (D if D.dim() == 2 else D[:, None])
    a.D, a.D_stride = _ptr(Dm), _st(Dm, 2)
    a.z, a.z_stride = _ptr(z), _st(z, 4)
    a.dt_bias = _ptr(dt_bias)
    a.dt_bias_stride = dt_bias.stride(0) if dt_bias is not None else 0
    a.initial_states, a.initial_states_stride = _ptr(initial_states), _st(initial_states, 4)
    a.seq_idx, a.seq_idx_stride = _ptr(seq_idx), _st(seq_idx, 2)


def ssd_forward(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None, initial_states=None,
                seq_idx=None, dt_softplus=False, dt_limit=(0.0, float("inf")),
                want_final_states=False, want_out_x=False, kernel_events=None, cu_seqlens=None):
    """One forward launch sequence.  Returns (out, out_x, final_states, varlen_states); out_x
    (the output before the z gate) only with z and ``want_out_x``, final_states only when
    asked, varlen_states [nseq, nheads, headdim, dstate] (x's dtype) only with
    ``cu_seqlens`` (batch 1; chunk_state_varlen, ssd_chunk_state.py:884-910).
    ``kernel_events``: optional pair of torch.cuda.Events that the library records right
    before and after its chunk-scan kernel (measurement only)."""
    batch, seqlen, nheads, headdim = x.shape
    dstate = B.shape[-1]
    x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx = _prepare(
        x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx)
    dtype = x.dtype
    with torch.cuda.device(x.device):
        out = torch.empty(x.shape, dtype=dtype, device=x.device)
        out_x = torch.empty_like(out) if (z is not None and want_out_x) else None
        final = (torch.empty(batch, nheads, headdim, dstate, dtype=torch.float32, device=x.device)
                 if want_final_states else None)
        a = _lib.S6SsdFwdArgs()
        a.p = _problem(x, B, chunk_size, D, z, dt_bias, initial_states, seq_idx, dt_softplus,
                       dt_limit)
        _fill_inputs(a, x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx)
        a.out, a.out_stride = _ptr(out), _st(out, 4)
        a.out_x, a.out_x_stride = _ptr(out_x), _st(out_x, 4)
        a.final_states = _ptr(final)
        varlen = None
        if cu_seqlens is not None:
            cu = cu_seqlens.to(device=x.device, dtype=torch.int32).contiguous()
            varlen = torch.empty(cu.numel() - 1, nheads, headdim, dstate, dtype=dtype,
                                 device=x.device)
            a.cu_seqlens, a.nseq, a.varlen_states = _ptr(cu), cu.numel() - 1, _ptr(varlen)
        nbytes = _lib.LIB.s6_ssd_fwd_workspace_bytes(ctypes.byref(a.p))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        a.workspace, a.workspace_bytes = _ptr(ws), nbytes
        if kernel_events is not None:
            a.kernel_events[0], a.kernel_events[1] = (e.cuda_event for e in kernel_events)
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check(_lib.LIB.s6_ssd_fwd(ctypes.byref(a), ctypes.c_void_p(stream)), "s6_ssd_fwd")
    return out, out_x, final, varlen


def ssd_backward(dout, x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                 initial_states=None, seq_idx=None, dt_softplus=False,
                 dt_limit=(0.0, float("inf")), out_x=None, dfinal_states=None):
    """One backward launch sequence (recomputing the forward's chunk quantities).  Returns
    (dx, ddt, dA, dB, dC, dD, dz, ddt_bias, dinitial_states) in the dtypes of the inputs
    they belong to; None for absent inputs."""
    x0, dt0, A0, B0, C0, D0, z0, bias0, init0 = x, dt, A, B, C, D, z, dt_bias, initial_states
    x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx = _prepare(
        x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx)
    dtype = x.dtype
    dout = _rows16(dout.to(dtype))
    if z is not None:
        assert out_x is not None, "the z gate's backward needs the forward's pre-gate output"
        out_x = out_x.to(dtype)
    batch, seqlen, nheads, headdim = x.shape
    dev = x.device
    with torch.cuda.device(dev):
        dx = torch.empty(x.shape, dtype=dtype, device=dev)
        ddt = torch.empty(dt.shape, dtype=dtype, device=dev)
        dA = torch.empty(nheads, dtype=torch.float32, device=dev)
        dB = torch.empty(B.shape, dtype=dtype, device=dev)
        dC = torch.empty(C.shape, dtype=dtype, device=dev)
        dD = torch.empty(D.shape, dtype=torch.float32, device=dev) if D is not None else None
        dz = torch.empty(z.shape, dtype=dtype, device=dev) if z is not None else None
        dbias = torch.empty(nheads, dtype=torch.float32, device=dev) if dt_bias is not None else None
        dinit = (torch.empty(initial_states.shape, dtype=torch.float32, device=dev)
                 if initial_states is not None else None)
        dfin = dfinal_states.float() if dfinal_states is not None else None
        a = _lib.S6SsdBwdArgs()
        a.p = _problem(x, B, chunk_size, D, z, dt_bias, initial_states, seq_idx, dt_softplus,
                       dt_limit)
        _fill_inputs(a, x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx)
        a.dout, a.dout_stride = _ptr(dout), _st(dout, 4)
        a.out_x, a.out_x_stride = _ptr(out_x if z is not None else None), _st(out_x if z is not None else None, 4)
        a.dfinal_states, a.dfinal_states_stride = _ptr(dfin), _st(dfin, 4)
        a.dx, a.dx_stride = _ptr(dx), _st(dx, 4)
        a.ddt, a.ddt_stride = _ptr(ddt), _st(ddt, 3)
        a.dA = _ptr(dA)
        a.dB, a.dB_stride = _ptr(dB), _st(dB, 4)
        a.dC, a.dC_stride = _ptr(dC), _st(dC, 4)
        a.dD = _ptr(dD)
        a.dz, a.dz_stride = _ptr(dz), _st(dz, 4)
        a.ddt_bias = _ptr(dbias)
        a.dinitial_states = _ptr(dinit)
        nbytes = _lib.LIB.s6_ssd_bwd_workspace_bytes(ctypes.byref(a.p))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = _ptr(ws), nbytes
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(_lib.LIB.s6_ssd_bwd(ctypes.byref(a), ctypes.c_void_p(stream)), "s6_ssd_bwd")
    like = lambda g, t: None if g is None else g.to(t.dtype)
    return (like(dx, x0), like(ddt, dt0), like(dA, A0), like(dB, B0), like(dC, C0),
            like(dD, D0) if D0 is not None else None, like(dz, z0) if z0 is not None else None,
            like(dbias, bias0) if bias0 is not None else None,
            like(dinit, init0) if init0 is not None else None)


class MambaChunkScanCombinedFn(torch.autograd.Function):
    """Autograd boundary with the reference's 16 inputs (ssd_combined.py:532-560)."""

    @staticmethod
    def forward(ctx, x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                initial_states=None, seq_idx=None, cu_seqlens=None, dt_softplus=False,
                dt_limit=(0.0, float("inf")), return_final_states=False,
                return_varlen_states=False):
        # the reference's argument rules (ssd_combined.py:537-540, 329)
        if not return_varlen_states:
            cu_seqlens = None
        else:
            assert cu_seqlens is not None, "cu_seqlens must be provided if return_varlen_states is True"
            assert x.shape[0] == 1, \
                "passing cu_seqlens to get the varlen states is only supported if batch dimension is 1"
        out, out_x, final, varlen = ssd_forward(
            x, dt, A, B, C, chunk_size, D=D, z=z, dt_bias=dt_bias, initial_states=initial_states,
            seq_idx=seq_idx, dt_softplus=dt_softplus, dt_limit=dt_limit,
            want_final_states=return_final_states, want_out_x=z is not None,
            cu_seqlens=cu_seqlens)
        ctx.save_for_backward(x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx, out_x)
        ctx.chunk_size, ctx.dt_softplus, ctx.dt_limit = chunk_size, dt_softplus, dt_limit
        ctx.return_final_states = return_final_states
        ctx.return_varlen_states = return_varlen_states
        if not return_varlen_states:
            return out if not return_final_states else (out, final)
        return (out, varlen) if not return_final_states else (out, final, varlen)

    @staticmethod
    def backward(ctx, dout, *args):
        assert not ctx.return_varlen_states, "return_varlen_states is not supported in backward"
        x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx, out_x = ctx.saved_tensors
        dfinal = args[0] if ctx.return_final_states else None
        dx, ddt, dA, dB, dC, dD, dz, dbias, dinit = ssd_backward(
            dout, x, dt, A, B, C, ctx.chunk_size, D=D, z=z, dt_bias=dt_bias,
            initial_states=initial_states, seq_idx=seq_idx, dt_softplus=ctx.dt_softplus,
            dt_limit=ctx.dt_limit, out_x=out_x, dfinal_states=dfinal)
        return (dx, ddt, dA, dB, dC, None, dD, dz, dbias, dinit, None, None, None, None, None,
                None)


def mamba_chunk_scan_combined(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                              initial_states=None, seq_idx=None, cu_seqlens=None,
                              dt_softplus=False, dt_limit=(0.0, float("inf")),
                              return_final_states=False, return_varlen_states=False):
    return MambaChunkScanCombinedFn.apply(x, dt, A, B, C, chunk_size, D, z, dt_bias,
                                          initial_states, seq_idx, cu_seqlens, dt_softplus,
                                          dt_limit, return_final_states, return_varlen_states)
