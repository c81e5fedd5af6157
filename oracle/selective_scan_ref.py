"""CPU restatement of the reference S6 selective scan -- TEST INFRASTRUCTURE ONLY.

This module is the parity oracle.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it, and only as the checker (or, for the
CPU baseline, as the thing timed on the host).  The product path (``s6scan``) never
imports anything under ``oracle/``.

``selective_scan_ref`` restates, op for op and in the same order, the reference's
``selective_scan_ref``
(/root/reference/zoology/zoology/mixers/mamba_ssm/ops/selective_scan_interface.py:91-157):

* upcast ``u``/``delta`` to fp32, add ``delta_bias``, ``F.softplus`` (threshold 20)  (107-112)
* ``deltaA = exp(einsum('bdl,dn->bdln'))``                                          (126)
* ``deltaB_u = einsum('bdl,bnl,bdl->bdln')`` or the grouped ``bdnl`` form            (127-134)
* sequential loop ``x = deltaA[:,:,i]*x + deltaB_u[:,:,i]``; ``y = einsum(x, C_i)``   (138-151)
* ``out = y + u*D``; ``out *= silu(z)``; ``out.to(dtype_in)``                         (152-157)

The complex-A branch (116-121, 149-150) and the time-invariant 2-D B/C branch (127-128,
140-141) are out of scope for the GPU path; they are kept here so the oracle is a complete
restatement, and the GPU interface rejects them.

Gradients: the reference computes its CPU gradients with autograd through this same
function, so the oracle does too (``torch.autograd.grad`` over ``selective_scan_ref``).

Varlen: ``selective_scan_ref_varlen`` restates the packed-sequence convention used by the
reference's chunked scans (the state is reset to zero where ``seq_idx`` changes,
/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/ssd_state_passing.py:76-78,
and ``cu_seqlens`` offsets, ssd_combined.py:326-332) as independent per-segment calls.

Pinned by ``tests/test_oracle.py`` against a float64 brute force (``oracle/brute64.py``),
closed forms (L=1, geometric series, Delta=0, abar=0, N=1) and invariants (chunk split,
linearity in u, group broadcast, varlen == per-segment, layout).
"""
import torch
import torch.nn.functional as F


def _repeat_groups(t, dim):
    # einops ``repeat(t, "B G N L -> B (G H) N L", H=dim // G)``: G is the outer factor,
    # so each group is repeated H times consecutively (SSI:133, 136).
    return t.repeat_interleave(dim // t.shape[1], dim=1)


def selective_scan_ref(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                       delta_softplus=False, return_last_state=False, compute_dtype=torch.float32):
    """Restatement of SSI:91-157.  u, delta, z: [B, D, L]; A: [D, N];
    B, C: [B, N, L] or [B, G, N, L] (or [D, N] time-invariant); D, delta_bias: [D].

    ``compute_dtype`` is the reference's ``.float()`` (fp32); float64 is used only by the
    tests that pin this restatement with ``gradcheck``."""
    dtype_in = u.dtype
    cf = lambda t: t.to(compute_dtype)
    u = cf(u)
    delta = cf(delta)
    if delta_bias is not None:
        delta = delta + cf(delta_bias[..., None])
    if delta_softplus:
        delta = F.softplus(delta)
    batch, dim, dstate = u.shape[0], A.shape[0], A.shape[1]
    is_variable_B = B.dim() >= 3
    is_variable_C = C.dim() >= 3
    if A.is_complex():
        if is_variable_B:
            B = torch.view_as_complex(cf(B).unflatten(-1, (-1, 2)))
        if is_variable_C:
            C = torch.view_as_complex(cf(C).unflatten(-1, (-1, 2)))
    else:
        B = cf(B)
        C = cf(C)
    x = A.new_zeros((batch, dim, dstate))
    ys = []
    deltaA = torch.exp(torch.einsum('bdl,dn->bdln', delta, A))
    if not is_variable_B:
        deltaB_u = torch.einsum('bdl,dn,bdl->bdln', delta, B, u)
    else:
        if B.dim() == 3:
            deltaB_u = torch.einsum('bdl,bnl,bdl->bdln', delta, B, u)
        else:
            B = _repeat_groups(B, dim)
            deltaB_u = torch.einsum('bdl,bdnl,bdl->bdln', delta, B, u)
    if is_variable_C and C.dim() == 4:
        C = _repeat_groups(C, dim)
    last_state = None
    for i in range(u.shape[2]):
        x = deltaA[:, :, i] * x + deltaB_u[:, :, i]
        if not is_variable_C:
            y = torch.einsum('bdn,dn->bd', x, C)
        else:
            if C.dim() == 3:
                y = torch.einsum('bdn,bn->bd', x, C[:, :, i])
            else:
                y = torch.einsum('bdn,bdn->bd', x, C[:, :, :, i])
        if i == u.shape[2] - 1:
            last_state = x
        if y.is_complex():
            y = y.real * 2
        ys.append(y)
    y = torch.stack(ys, dim=2)  # (batch dim L)
    out = y if D is None else y + u * D.unsqueeze(-1)
    if z is not None:
        out = out * F.silu(z)
    out = out.to(dtype=dtype_in)
    return out if not return_last_state else (out, last_state)


def selective_scan_ref_varlen(u, delta, A, B, C, cu_seqlens, D=None, z=None, delta_bias=None,
                              delta_softplus=False, return_last_state=False,
                              compute_dtype=torch.float32):
    """Packed variable-length scan: batch 1, sequences [cu[i], cu[i+1]) scanned
    independently from a zero state.  Returns out [1, D, T] and, if asked, the
    per-sequence final states [nseq, D, N] (fp32; zero for an empty sequence)."""
    assert u.shape[0] == 1
    cu = [int(v) for v in cu_seqlens.tolist()]
    outs, states = [], []
    for s, e in zip(cu[:-1], cu[1:]):
        if e == s:  # an empty sequence produces no output and a zero final state
            states.append(A.new_zeros((1, A.shape[0], A.shape[1]), dtype=compute_dtype))
            continue
        sl = slice(s, e)
        sub = lambda t: None if t is None else t[..., sl]
        res = selective_scan_ref(u[..., sl], delta[..., sl], A, B[..., sl], C[..., sl], D=D,
                                 z=sub(z), delta_bias=delta_bias, delta_softplus=delta_softplus,
                                 return_last_state=True, compute_dtype=compute_dtype)
        outs.append(res[0])
        states.append(res[1])
    out = torch.cat(outs, dim=-1)
    if return_last_state:
        return out, torch.cat(states, dim=0)
    return out


def selective_scan_ref_grads(u, delta, A, B, C, D, dout, z=None, delta_bias=None,
                             delta_softplus=False, cu_seqlens=None, compute_dtype=torch.float32):
    """Gradients of ``(out * dout).sum()`` by autograd through the restatement, as the
    reference obtains them for its CPU path.  Returns a dict with keys
    du, ddelta, dA, dB, dC, dD, dz, ddelta_bias (None where the input is None)."""
    leaves = dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=delta_bias)
    req = {k: v.detach().clone().requires_grad_(True) for k, v in leaves.items() if v is not None}
    args = {k: req.get(k) for k in leaves}
    if cu_seqlens is None:
        out = selective_scan_ref(args['u'], args['delta'], args['A'], args['B'], args['C'],
                                 D=args['D'], z=args['z'], delta_bias=args['delta_bias'],
                                 delta_softplus=delta_softplus, compute_dtype=compute_dtype)
    else:
        out = selective_scan_ref_varlen(args['u'], args['delta'], args['A'], args['B'], args['C'],
                                        cu_seqlens, D=args['D'], z=args['z'],
                                        delta_bias=args['delta_bias'],
                                        delta_softplus=delta_softplus,
                                        compute_dtype=compute_dtype)
    keys = list(req.keys())
    grads = torch.autograd.grad((out.double() * dout.double()).sum(), [req[k] for k in keys])
    res = {('d' + k): None for k in leaves}
    for k, g in zip(keys, grads):
        res['d' + k] = g
    return res
