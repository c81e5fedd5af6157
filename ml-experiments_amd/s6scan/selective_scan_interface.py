"""Drop-in S6 selective scan for MI355X.

Same call signature and return conventions as the reference's ``SelectiveScanFn`` /
``selective_scan_fn`` (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/
selective_scan_interface.py:19-88):

    selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                      delta_softplus=False, return_last_state=False)
        -> out | (out, last_state)

* u, delta, z: [batch, dim, seqlen] (any strides -- channel-last views such as
  ``x.mT`` are used in place, no ``.contiguous()`` copy); A: [dim, dstate] fp32;
  B, C: [batch, dstate, seqlen] or [batch, ngroups, dstate, seqlen]; D, delta_bias: [dim].
* out has u's dtype; with z it is ``(y + D u) * silu(z)``; last_state is fp32
  [batch, dim, dstate] and, as in the reference, carries no gradient (SSI:84-87).
* Backward returns the reference's 10-slot tuple (SSI:74-79).

Extension: keyword-only ``cu_seqlens`` (int32 [nseq+1], batch must be 1) scans packed
variable-length sequences with the state reset at every sequence start; last_state is
then [nseq, dim, dstate].

All work runs in the HIP kernels of ``libs6scan.so`` through its C ABI.  There is no CPU
or PyTorch fallback: inputs that are not on a ROCm device raise ``RuntimeError``, and the
reference's complex-A and time-invariant-B/C variants raise ``NotImplementedError``.
"""
import ctypes
import os

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _strides(t, n):
    if t is None:
        return (0,) * n
    return tuple(t.stride())


def check_cu_seqlens(cu_seqlens, seqlen):
    """Contents of packed-varlen offsets: cu[0] == 0, non-decreasing, cu[-1] == seqlen (the
    convention of the reference's varlen chunked scan, ssd_combined.py:576-577 and
    ssd_state_passing.py:76-78).  Reads the nseq + 1 offsets to the host once (a device
    synchronisation) and checks them with the library's host-only validator; a malformed
    vector raises ValueError and is never passed to a kernel."""
    host = cu_seqlens.detach().to("cpu", torch.int32).contiguous()
    rc = _lib.LIB.s6_validate_cu_seqlens(ctypes.c_void_p(host.data_ptr()), host.numel() - 1,
                                         int(seqlen))
    if rc != _lib.OK:
        raise ValueError(f"s6scan: {_lib.last_error()}")


def check_inputs(u, delta, A, B, C, D=None, z=None, delta_bias=None, cu_seqlens=None):
    """Shape/dtype/device checks of the reference contract; returns the problem tuple
    (batch, dim, seqlen, dstate, ngroups, nseq).  Pure host logic: runs without a GPU."""
    if A.is_complex():
        raise NotImplementedError("s6scan: complex A is not supported (SSI:116-121)")
    if B.dim() < 3 or C.dim() < 3:
        raise NotImplementedError(
            "s6scan: time-invariant B/C ([dim, dstate]) are not supported (SSI:127-128)")
    if u.dim() != 3:
        raise ValueError(f"u must be [batch, dim, seqlen], got shape {tuple(u.shape)}")
    batch, dim, seqlen = u.shape
    if delta.shape != u.shape:
        raise ValueError(f"delta shape {tuple(delta.shape)} != u shape {tuple(u.shape)}")
    if u.dtype not in _DTYPES:
        raise TypeError(f"u dtype {u.dtype} not supported (float32, bfloat16, float16)")
    if delta.dtype != u.dtype:
        raise TypeError(f"delta dtype {delta.dtype} must equal u dtype {u.dtype}")
    if A.dim() != 2 or A.shape[0] != dim:
        raise ValueError(f"A must be [dim={dim}, dstate], got {tuple(A.shape)}")
    if A.dtype != torch.float32:
        raise TypeError(f"A must be float32, got {A.dtype}")
    dstate = A.shape[1]
    shapes = []
    for name, M in (("B", B), ("C", C)):
        if M.dim() not in (3, 4):
            raise ValueError(f"{name} must be [batch, dstate, seqlen] or [batch, G, dstate, seqlen]")
        G = 1 if M.dim() == 3 else M.shape[1]
        want = (batch, dstate, seqlen) if M.dim() == 3 else (batch, G, dstate, seqlen)
        if tuple(M.shape) != want:
            raise ValueError(f"{name} shape {tuple(M.shape)} != expected {want}")
        if M.dtype not in (u.dtype, torch.float32):
            raise TypeError(f"{name} dtype {M.dtype} must be u's dtype or float32")
        shapes.append(G)
    if shapes[0] != shapes[1]:
        raise ValueError("B and C must have the same number of groups")
    if B.dtype != C.dtype:
        raise TypeError("B and C must have the same dtype")
    G = shapes[0]
    if dim % G != 0:
        raise ValueError(f"dim {dim} must be divisible by the number of groups {G}")
    if D is not None and (D.shape != (dim,) or D.dtype != torch.float32):
        raise ValueError("D must be float32 [dim]")
    if delta_bias is not None and (delta_bias.shape != (dim,) or delta_bias.dtype != torch.float32):
        raise ValueError("delta_bias must be float32 [dim]")
    if z is not None:
        if z.shape != u.shape:
            raise ValueError(f"z shape {tuple(z.shape)} != u shape {tuple(u.shape)}")
        if z.dtype != u.dtype:
            raise TypeError(f"z dtype {z.dtype} must equal u dtype {u.dtype}")
    nseq = 0
    if cu_seqlens is not None:
        if batch != 1:
            raise ValueError("cu_seqlens requires batch == 1 (packed sequences)")
        if cu_seqlens.dim() != 1 or cu_seqlens.dtype != torch.int32 or cu_seqlens.numel() < 2:
            raise ValueError("cu_seqlens must be an int32 vector [nseq+1]")
        nseq = cu_seqlens.numel() - 1
        check_cu_seqlens(cu_seqlens, seqlen)
    if dstate > _lib.MAX_DSTATE_FWD:
        raise NotImplementedError(f"s6scan: dstate {dstate} > {_lib.MAX_DSTATE_FWD} is not supported")
    tensors = [t for t in (u, delta, A, B, C, D, z, delta_bias, cu_seqlens) if t is not None]
    dev = u.device
    if dev.type != "cuda":
        raise RuntimeError("s6scan runs on ROCm devices only; got tensors on " + str(dev))
    for t in tensors:
        if t.device != dev:
            raise RuntimeError("all s6scan inputs must be on the same device")
    return batch, dim, seqlen, dstate, G, nseq


def _problem(u, B, z, D, delta_bias, delta_softplus, dims):
    batch, dim, seqlen, dstate, G, nseq = dims
    return _lib.S6Problem(batch, dim, seqlen, dstate, G, _DTYPES[u.dtype], _DTYPES[B.dtype],
                          int(D is not None), int(z is not None), int(delta_bias is not None),
                          int(bool(delta_softplus)), nseq)


def _dense(t):
    """True when t's elements exactly fill a block of memory (any dimension order)."""
    expect = 1
    for i in sorted(range(t.dim()), key=lambda i: t.stride(i)):
        if t.size(i) != 1 and t.stride(i) != expect:
            return False
        expect *= t.size(i)
    return True


def _empty_like(t, u):
    """A new tensor of t's shape and dtype in t's layout, or in u's (same shape) when t is a
    strided view (e.g. a half of a channel-last [B, L, 2D] buffer) that empty_like would
    turn into an L-contiguous tensor."""
    return torch.empty_like(t) if _dense(t) else torch.empty_like(u, dtype=t.dtype)


def _check_out(t, like, name):
    if t.shape != like.shape or t.dtype != like.dtype or t.device != like.device:
        raise ValueError(f"{name} must have shape {tuple(like.shape)}, dtype {like.dtype} "
                         f"and device {like.device}")
    return t


def _as4(M):
    return M.unsqueeze(1) if M.dim() == 3 else M


def _events(kernel_events):
    """Raw hipEvent_t handles of a (torch.cuda.Event, torch.cuda.Event) pair, or NULLs."""
    if kernel_events is None:
        return (None, None)
    return tuple(ctypes.c_void_p(e.cuda_event) for e in kernel_events)


def _ckpt_check(x_ckpt, batch, nck, dim, dstate, device):
    want = (batch, nck, dim, dstate)
    if (tuple(x_ckpt.shape) != want or x_ckpt.dtype != torch.float32
            or x_ckpt.device != device or (dstate > 1 and x_ckpt.stride(3) != 1)):
        raise ValueError(f"x_ckpt must be a float32 view of shape {want} on {device} "
                         "with unit dstate stride")
    return x_ckpt


def _ckpt_strides(x_ckpt):
    # the dstate axis is contiguous (a size-1 axis may carry any stride in torch)
    return (0,) * 4 if x_ckpt is None else tuple(x_ckpt.stride()[:3]) + (1,)


def _fwd_args(prob, u, delta, A, B4, C4, D, z, delta_bias, cu_seqlens, out, out_z, x_ckpt,
              last_state):
    args = _lib.S6FwdArgs()
    args.p = prob
    args.u, args.u_stride = _ptr(u), _strides(u, 3)
    args.delta, args.delta_stride = _ptr(delta), _strides(delta, 3)
    args.A, args.A_stride = _ptr(A), _strides(A, 2)
    args.B, args.B_stride = _ptr(B4), _strides(B4, 4)
    args.C, args.C_stride = _ptr(C4), _strides(C4, 4)
    args.D, args.D_stride = _ptr(D), (D.stride(0) if D is not None else 0)
    args.z, args.z_stride = _ptr(z), _strides(z, 3)
    args.delta_bias = _ptr(delta_bias)
    args.delta_bias_stride = delta_bias.stride(0) if delta_bias is not None else 0
    args.cu_seqlens = _ptr(cu_seqlens)
    args.out, args.out_stride = _ptr(out), _strides(out, 3)
    args.out_z, args.out_z_stride = _ptr(out_z), _strides(out_z, 3)
    args.x_ckpt, args.x_ckpt_stride = _ptr(x_ckpt), _ckpt_strides(x_ckpt)
    args.last_state = _ptr(last_state)
    return args


_FWD_KERNELS = {0: "chunked", 1: "chunked_rows", 2: "single_pass"}


def forward_kernel(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                   cu_seqlens=None):
    """The forward kernels selective_scan_forward runs on these tensors, outputs laid out like
    u as it allocates them (``s6_fwd_kernel``): "single_pass", "chunked_rows" (the chunked
    kernels with whole 8-step row blocks per lane) or "chunked" (one step at a time).  Host
    only: no kernel runs and nothing is allocated on the device."""
    dims = check_inputs(u, delta, A, B, C, D, z, delta_bias, cu_seqlens)
    prob = _problem(u, B, z, D, delta_bias, delta_softplus, dims)
    args = _fwd_args(prob, u, delta, A, _as4(B), _as4(C), D, z, delta_bias, cu_seqlens, u,
                     u if z is not None else None, None, None)
    # The outputs stand in as u's pointer with the strides empty_like(u) gives them; only
    # their layout and alignment enter the choice, which needs u aligned as well.
    like = _strides(torch.empty_like(u, device="meta"), 3)
    args.out_stride = like
    if z is not None:
        args.out_z_stride = like
    rc = _lib.LIB.s6_fwd_kernel(ctypes.byref(args))
    if rc < 0:
        _lib.check(rc, "s6_fwd_kernel")
    return _FWD_KERNELS[rc]


def selective_scan_forward(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                           delta_softplus=False, cu_seqlens=None, want_ckpt=True,
                           want_last_state=False, kernel_events=None, x_ckpt_out=None,
                           no_alloc=False):
    """One forward launch.  Returns (out, out_z, x_ckpt, last_state); out_z is None without
    z, x_ckpt is None unless ``want_ckpt``, last_state is None unless ``want_last_state``.
    ``x_ckpt_out``: optional preallocated checkpoint view [batch, nck, dim, dstate] fp32 with
    a unit dstate stride and any other strides (nck = ceil(seqlen / 8)), written in place of
    a new contiguous one.
    ``kernel_events``: optional pair of already-recorded torch.cuda.Events that the library
    re-records around its main scan kernel (measurement only).
    ``no_alloc``: run ``s6_fwd_noalloc``, whose workspace is the library's per-device scratch
    array, so the call allocates no device workspace (outputs are still new tensors unless
    preallocated)."""
    dims = check_inputs(u, delta, A, B, C, D, z, delta_bias, cu_seqlens)
    batch, dim, seqlen, dstate, G, nseq = dims
    prob = _problem(u, B, z, D, delta_bias, delta_softplus, dims)
    B4, C4 = _as4(B), _as4(C)
    with torch.cuda.device(u.device):
        out = torch.empty_like(u)
        out_z = torch.empty_like(u) if z is not None else None
        nck = _lib.LIB.s6_num_checkpoints(ctypes.byref(prob))
        if x_ckpt_out is not None:
            x_ckpt = _ckpt_check(x_ckpt_out, batch, nck, dim, dstate, u.device)
        else:
            x_ckpt = (torch.empty(batch, nck, dim, dstate, dtype=torch.float32, device=u.device)
                      if want_ckpt else None)
        nls = nseq if nseq > 0 else batch
        last_state = (torch.empty(nls, dim, dstate, dtype=torch.float32, device=u.device)
                      if want_last_state else None)
        args = _fwd_args(prob, u, delta, A, B4, C4, D, z, delta_bias, cu_seqlens, out, out_z,
                         x_ckpt, last_state)
        args.kernel_events = _events(kernel_events)
        stream = torch.cuda.current_stream(u.device).cuda_stream
        if no_alloc:
            args.workspace, args.workspace_bytes = None, 0
            _lib.check(_lib.LIB.s6_fwd_noalloc(ctypes.byref(args), ctypes.c_void_p(stream)),
                       "s6_fwd_noalloc")
        else:
            nbytes = _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(prob))
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=u.device)
            args.workspace, args.workspace_bytes = _ptr(ws), nbytes
            _lib.check(_lib.LIB.s6_fwd(ctypes.byref(args), ctypes.c_void_p(stream)), "s6_fwd")
    return out, out_z, x_ckpt, last_state


def backward_row_blocks(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, out=None,
                        cu_seqlens=None, recompute_out_z=False):
    """True if selective_scan_backward on these tensors (its outputs laid out as it allocates
    them) runs the row-block kernels (``s6_bwd_row_blocks``).  Host only."""
    dims = check_inputs(u, delta, A, B, C, D, z, delta_bias, cu_seqlens)
    prob = _problem(u, B, z, D, delta_bias, delta_softplus, dims)
    args = _lib.S6BwdArgs()
    args.p = prob
    meta = lambda t: _strides(torch.empty_like(t, device="meta") if _dense(t)
                              else torch.empty_like(u, dtype=t.dtype, device="meta"), 3)
    args.u, args.u_stride = _ptr(u), _strides(u, 3)
    args.delta, args.delta_stride = _ptr(delta), _strides(delta, 3)
    args.dout, args.dout_stride = _ptr(dout), _strides(dout, 3)
    args.z, args.z_stride = _ptr(z), _strides(z, 3)
    args.out, args.out_stride = _ptr(out), _strides(out, 3)
    # the outputs stand in as u's pointer (their layout and alignment enter the choice)
    args.du, args.du_stride = _ptr(u), meta(u)
    args.ddelta, args.ddelta_stride = _ptr(u), meta(delta)
    if z is not None:
        args.dz, args.dz_stride = _ptr(u), meta(z)
        if recompute_out_z:
            args.out_z, args.out_z_stride = _ptr(u), meta(z)
    rc = _lib.LIB.s6_bwd_row_blocks(ctypes.byref(args))
    if rc < 0:
        _lib.check(rc, "s6_bwd_row_blocks")
    return rc == 1


def selective_scan_backward(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, x_ckpt,
                            out=None, cu_seqlens=None, kernel_events=None, du_out=None,
                            dz_out=None, recompute_out_z=False):
    """One backward launch.  Returns (du, ddelta, dA, dB, dC, dD, dz, ddelta_bias) with dB, dC
    in B/C's own rank (3-D or 4-D) and fp32 like the reference kernel's; None for absent
    inputs.  ``du_out`` / ``dz_out``: optional preallocated outputs of u's / z's shape and
    dtype (any strides), as the reference kernel's ``dz`` argument (SSI:263-267).  With
    ``recompute_out_z`` (z given) a 9th element ``out_z = out * silu(z)`` is returned, the
    reference's recompute_out_z output."""
    dims = check_inputs(u, delta, A, B, C, D, z, delta_bias, cu_seqlens)
    batch, dim, seqlen, dstate, G, nseq = dims
    if dstate > _lib.MAX_DSTATE_BWD:
        raise NotImplementedError(
            f"s6scan: backward supports dstate <= {_lib.MAX_DSTATE_BWD}, got {dstate}")
    prob = _problem(u, B, z, D, delta_bias, delta_softplus, dims)
    B4, C4 = _as4(B), _as4(C)
    if dout.shape != u.shape:
        raise ValueError("dout must have u's shape")
    if dout.dtype != u.dtype:
        dout = dout.to(u.dtype)
    with torch.cuda.device(u.device):
        du = torch.empty_like(u) if du_out is None else _check_out(du_out, u, "du_out")
        ddelta = _empty_like(delta, u)
        dA = torch.empty(dim, dstate, dtype=torch.float32, device=u.device)
        dB4 = torch.empty(B4.shape, dtype=torch.float32, device=u.device)
        dC4 = torch.empty(C4.shape, dtype=torch.float32, device=u.device)
        dD = torch.empty(dim, dtype=torch.float32, device=u.device) if D is not None else None
        dz = None
        if z is not None:
            dz = _empty_like(z, u) if dz_out is None else _check_out(dz_out, z, "dz_out")
        out_z = _empty_like(z, u) if (z is not None and recompute_out_z) else None
        dbias = (torch.empty(dim, dtype=torch.float32, device=u.device)
                 if delta_bias is not None else None)
        args = _lib.S6BwdArgs()
        args.p = prob
        args.u, args.u_stride = _ptr(u), _strides(u, 3)
        args.delta, args.delta_stride = _ptr(delta), _strides(delta, 3)
        args.A, args.A_stride = _ptr(A), _strides(A, 2)
        args.B, args.B_stride = _ptr(B4), _strides(B4, 4)
        args.C, args.C_stride = _ptr(C4), _strides(C4, 4)
        args.D, args.D_stride = _ptr(D), (D.stride(0) if D is not None else 0)
        args.z, args.z_stride = _ptr(z), _strides(z, 3)
        args.delta_bias = _ptr(delta_bias)
        args.delta_bias_stride = delta_bias.stride(0) if delta_bias is not None else 0
        args.cu_seqlens = _ptr(cu_seqlens)
        args.dout, args.dout_stride = _ptr(dout), _strides(dout, 3)
        nck = _lib.LIB.s6_num_checkpoints(ctypes.byref(prob))
        _ckpt_check(x_ckpt, batch, nck, dim, dstate, u.device)
        args.x_ckpt, args.x_ckpt_stride = _ptr(x_ckpt), _ckpt_strides(x_ckpt)
        args.out, args.out_stride = _ptr(out), _strides(out, 3)
        args.du, args.du_stride = _ptr(du), _strides(du, 3)
        args.ddelta, args.ddelta_stride = _ptr(ddelta), _strides(ddelta, 3)
        args.dA, args.dA_stride = _ptr(dA), _strides(dA, 2)
        args.dB, args.dB_stride = _ptr(dB4), _strides(dB4, 4)
        args.dC, args.dC_stride = _ptr(dC4), _strides(dC4, 4)
        args.dD, args.dD_stride = _ptr(dD), (dD.stride(0) if dD is not None else 0)
        args.dz, args.dz_stride = _ptr(dz), _strides(dz, 3)
        args.out_z, args.out_z_stride = _ptr(out_z), _strides(out_z, 3)
        args.ddelta_bias = _ptr(dbias)
        args.ddelta_bias_stride = dbias.stride(0) if dbias is not None else 0
        nbytes = _lib.LIB.s6_bwd_workspace_bytes(ctypes.byref(prob))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=u.device)
        args.workspace, args.workspace_bytes = _ptr(ws), nbytes
        args.kernel_events = _events(kernel_events)
        stream = torch.cuda.current_stream(u.device).cuda_stream
        _lib.check(_lib.LIB.s6_bwd(ctypes.byref(args), ctypes.c_void_p(stream)), "s6_bwd")
    dB = dB4.squeeze(1) if B.dim() == 3 else dB4
    dC = dC4.squeeze(1) if C.dim() == 3 else dC4
    if out_z is not None:
        return du, ddelta, dA, dB, dC, dD, dz, dbias, out_z
    return du, ddelta, dA, dB, dC, dD, dz, dbias


def _recompute_default():
    """``S6_RECOMPUTE_STATES=1`` in the environment makes state recomputation the default
    for callers that cannot pass ``recompute_states`` (code written for the reference's
    signature)."""
    return os.environ.get("S6_RECOMPUTE_STATES", "0") not in ("", "0")


class SelectiveScanFn(torch.autograd.Function):
    """Autograd boundary with the reference's 10 positional inputs (SSI:19-79), plus an
    optional 11th, ``cu_seqlens``, for packed variable-length input, and a 12th,
    ``recompute_states``.

    By default the forward keeps the fp32 state after every 8th step ([B, ceil(L/8), D, N],
    8 bytes per (b, t, d) at N = 16) for the backward.  With ``recompute_states`` it keeps
    none.  The tensors held from forward to backward are then the inputs alone, as with
    the reference's kernel (whose ``x`` is [B, D, ceil(L/2048), 2N], SSI:45-50), and the
    backward first reruns the forward to regenerate the checkpoints.  The gradients are the
    same bit for bit; the price is one more forward per backward."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                return_last_state=False, cu_seqlens=None, recompute_states=None):
        need_grad = any(ctx.needs_input_grad[:8])
        recompute = _recompute_default() if recompute_states is None else bool(recompute_states)
        out, out_z, x_ckpt, last_state = selective_scan_forward(
            u, delta, A, B, C, D, z, delta_bias, delta_softplus, cu_seqlens=cu_seqlens,
            want_ckpt=need_grad and not recompute, want_last_state=bool(return_last_state))
        ctx.delta_softplus = delta_softplus
        ctx.has_z = z is not None
        ctx.recompute = need_grad and recompute
        if ctx.recompute:
            x_ckpt = None
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, x_ckpt,
                              out if (z is not None and not ctx.recompute) else None,
                              cu_seqlens)
        res = out_z if z is not None else out
        if return_last_state:
            ctx.mark_non_differentiable(last_state)
            return res, last_state
        return res

    @staticmethod
    def backward(ctx, dout, *args):
        u, delta, A, B, C, D, z, delta_bias, x_ckpt, out, cu_seqlens = ctx.saved_tensors
        if ctx.recompute:
            # the same forward launches as a checkpointing forward: identical checkpoints
            out_r, _, x_ckpt, _ = selective_scan_forward(
                u, delta, A, B, C, D, z, delta_bias, ctx.delta_softplus, cu_seqlens=cu_seqlens,
                want_ckpt=True)
            out = out_r if z is not None else None
        if x_ckpt is None:
            raise RuntimeError("s6scan: backward called but no checkpoint was saved in forward")
        du, ddelta, dA, dB, dC, dD, dz, dbias = selective_scan_backward(
            u, delta, A, B, C, D, z, delta_bias, ctx.delta_softplus, dout, x_ckpt, out=out,
            cu_seqlens=cu_seqlens)
        return (du, ddelta, dA, dB, dC, dD, dz, dbias, None, None, None, None)


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                      return_last_state=False, *, cu_seqlens=None, recompute_states=None):
    """if return_last_state is True, returns (out, last_state); last_state has shape
    (batch, dim, dstate) (or (nseq, dim, dstate) with cu_seqlens) and carries no gradient.
    ``recompute_states``: keep no state checkpoints from forward to backward and rerun the
    forward in the backward instead (``SelectiveScanFn``); None takes the
    ``S6_RECOMPUTE_STATES`` environment default (off)."""
    return SelectiveScanFn.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus,
                                 return_last_state, cu_seqlens, recompute_states)
