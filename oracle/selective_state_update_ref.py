"""CPU restatement of selective_state_update -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and the other checker legs named in ``oracle/selective_scan_ref.py``)
may import this module, as the checker of ``s6scan.selective_state_update``.

``selective_state_update_ref`` restates the reference's ``selective_state_update_ref``
(/root/reference/zoology/zoology/mixers/mamba_ssm/ops/triton/selective_state_update.py:
204-265) op for op:

* unsqueeze the head axis of 3-D / 2-D inputs                                      (219-236)
* ``dt = dt + dt_bias``; ``dt = softplus(dt)``                                      (250-252)
* ``dA = exp(dt[..., None] * A)``                                                   (253)
* B, C repeated over the heads of each group (``"b g n -> b (g h) n"``)             (254-255)
* ``state <- state * dA + (dt * B) * x``  (in place)                                (256-257)
* ``out = einsum("bhdn,bhn->bhd", state, C)``; ``+ x * D``; ``* silu(z)``           (258-261)

One point follows the reference's kernel rather than its ``_ref`` function: ``out`` is
taken from the updated state at compute precision, before it is rounded to the state's
storage dtype (the kernel's order, :105-110; ``_ref`` rounds first, :257-258).  For an fp32
state the two are the same.

``compute_dtype`` runs the arithmetic in float64 for the pinning tests (the reference
computes in the tensors' own dtypes; fp32 here by default).  Pinned by
``tests/test_oracle_ssu.py``: L decode steps from a zero state reproduce the float64 scan
brute force (``brute64.scan_fwd64``: outputs and final state) for single- and multi-head
inputs; dt = 0 leaves the state unchanged; grouped B / C equal their explicit repeat.
"""
import torch
import torch.nn.functional as F


def selective_state_update_ref(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                               dt_softplus=False, compute_dtype=None):
    """Updates ``state`` in place and returns out (x's shape and dtype)."""
    has_heads = state.dim() > 3
    st = state if state.dim() == 4 else state.unsqueeze(1)
    x4 = x if x.dim() == 3 else x.unsqueeze(1)
    dt4 = dt if dt.dim() == 3 else dt.unsqueeze(1)
    A3 = A if A.dim() == 3 else A.unsqueeze(0)
    B3 = B if B.dim() == 3 else B.unsqueeze(1)
    C3 = C if C.dim() == 3 else C.unsqueeze(1)
    D2 = None if D is None else (D if D.dim() == 2 else D.unsqueeze(0))
    z4 = None if z is None else (z if z.dim() == 3 else z.unsqueeze(1))
    bias2 = None if dt_bias is None else (dt_bias if dt_bias.dim() == 2 else dt_bias.unsqueeze(0))
    batch, nheads, dim, dstate = st.shape
    ngroups = B3.shape[1]
    assert nheads % ngroups == 0
    cd = compute_dtype or torch.float32
    f = lambda t: None if t is None else t.to(cd)
    dtc = f(dt4)
    if bias2 is not None:
        dtc = dtc + f(bias2)
    dtc = F.softplus(dtc) if dt_softplus else dtc
    dA = torch.exp(dtc[..., None] * f(A3))                                 # (b, h, d, n)
    Bh = f(B3).repeat_interleave(nheads // ngroups, dim=1)                 # (b, h, n)
    Ch = f(C3).repeat_interleave(nheads // ngroups, dim=1)
    dB = dtc[..., None] * Bh[:, :, None, :]                                # (b, h, d, n)
    new = f(st) * dA + dB * f(x4)[..., None]
    st.copy_(new.to(st.dtype))
    out = torch.einsum("bhdn,bhn->bhd", new, Ch)
    if D2 is not None:
        out = out + f(x4) * f(D2)
    if z4 is not None:
        out = out * F.silu(f(z4))
    out = out.to(x.dtype)
    return out if has_heads else out.squeeze(1)
