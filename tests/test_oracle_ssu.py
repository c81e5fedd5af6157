"""Pins the selective_state_update restatement (oracle/selective_state_update_ref.py) on the
CPU: a run of decode steps is the scan (float64 brute force), dt = 0 is the identity on the
state, and grouped B / C equal their explicit repeat."""
import numpy as np
import pytest
import torch

from oracle.brute64 import scan_fwd64
from oracle.selective_state_update_ref import selective_state_update_ref


def _r(*s, g):
    return torch.randn(*s, generator=g, dtype=torch.float64)


@pytest.mark.parametrize("z_d_bias", [False, True])
def test_decode_steps_reproduce_the_scan(z_d_bias):
    g = torch.Generator().manual_seed(1)
    batch, dim, dstate, L = 2, 5, 4, 9
    u, dl = _r(batch, dim, L, g=g), _r(batch, dim, L, g=g) * 0.5
    A = -torch.exp(_r(dim, dstate, g=g))
    B, C = _r(batch, dstate, L, g=g), _r(batch, dstate, L, g=g)
    D = _r(dim, g=g) if z_d_bias else None
    z = _r(batch, dim, L, g=g) if z_d_bias else None
    bias = _r(dim, g=g) * 0.3 if z_d_bias else None
    want = scan_fwd64(u.numpy(), dl.numpy(), A.numpy(), B.numpy(), C.numpy(),
                      D=None if D is None else D.numpy(), z=None if z is None else z.numpy(),
                      delta_bias=None if bias is None else bias.numpy(), delta_softplus=True)
    state = torch.zeros(batch, dim, dstate, dtype=torch.float64)
    outs = []
    for t in range(L):
        outs.append(selective_state_update_ref(
            state, u[..., t], dl[..., t], A, B[..., t], C[..., t], D=D,
            z=None if z is None else z[..., t], dt_bias=bias, dt_softplus=True,
            compute_dtype=torch.float64))
    np.testing.assert_allclose(torch.stack(outs, -1).numpy(), want["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(state.numpy(), want["last_state"], rtol=1e-12, atol=1e-12)


def test_multihead_decode_is_the_scan_per_head():
    """(batch, nheads, dim) heads with grouped B / C: each head runs the scan with its
    group's B / C (heads h of group h // (nheads / ngroups))."""
    g = torch.Generator().manual_seed(2)
    batch, nheads, dim, dstate, ngroups, L = 2, 4, 3, 5, 2, 6
    u, dl = _r(batch, nheads, dim, L, g=g), _r(batch, nheads, dim, L, g=g) * 0.5
    A = -torch.exp(_r(nheads, dim, dstate, g=g))
    B, C = _r(batch, ngroups, dstate, L, g=g), _r(batch, ngroups, dstate, L, g=g)
    state = torch.zeros(batch, nheads, dim, dstate, dtype=torch.float64)
    outs = []
    for t in range(L):
        outs.append(selective_state_update_ref(state, u[..., t], dl[..., t], A, B[..., t],
                                               C[..., t], compute_dtype=torch.float64))
    out = torch.stack(outs, -1)
    for h in range(nheads):
        gi = h // (nheads // ngroups)
        want = scan_fwd64(u[:, h].numpy(), dl[:, h].numpy(), A[h].numpy(), B[:, gi].numpy(),
                          C[:, gi].numpy())
        np.testing.assert_allclose(out[:, h].numpy(), want["out"], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(state[:, h].numpy(), want["last_state"], rtol=1e-12, atol=1e-12)


def test_zero_dt_keeps_the_state():
    g = torch.Generator().manual_seed(3)
    state = _r(2, 3, 4, g=g)
    s0 = state.clone()
    x, A, B, C, D = _r(2, 3, g=g), -torch.exp(_r(3, 4, g=g)), _r(2, 4, g=g), _r(2, 4, g=g), _r(3, g=g)
    out = selective_state_update_ref(state, x, torch.zeros(2, 3, dtype=torch.float64), A, B, C,
                                     D=D, compute_dtype=torch.float64)
    torch.testing.assert_close(state, s0, rtol=0, atol=0)
    torch.testing.assert_close(out, torch.einsum("bdn,bn->bd", s0, C) + x * D)
