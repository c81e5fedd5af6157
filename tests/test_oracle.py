"""Pins the CPU oracle (the checker of every GPU parity test) without a GPU.

The reference ships no golden vectors or tests for the S6 scan, so the torch restatement
of selective_scan_ref is pinned by: an independent float64 brute force with a hand-derived
backward (oracle/brute64.py), torch.autograd.gradcheck, closed forms (L=1, geometric
series, Delta=0, abar=0, N=1) and invariants (causality, linearity in u, chunk-split state
passing, group broadcast, varlen == per-segment, layout).  The C restatement used for
full-size checks is pinned against both.  Each check is chosen so that a plausible slip
(dropped D term, B/C transposed, wrong softplus threshold, group repeat in the wrong
order, reset off by one step) fails it.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle.brute64 import scan_bwd64, scan_fwd64
from oracle.selective_scan_ref import (selective_scan_ref, selective_scan_ref_grads,
                                       selective_scan_ref_varlen)

F64 = torch.float64
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "s6_golden.npz")


def _inputs(B=2, D=6, L=9, N=4, G=1, seed=0, dtype=torch.float64, z=False, bias=False,
            positive_delta=True):
    g = torch.Generator("cpu").manual_seed(seed)
    u = torch.randn(B, D, L, generator=g, dtype=dtype)
    dl = torch.randn(B, D, L, generator=g, dtype=dtype) * 0.5
    if positive_delta and not bias:
        dl = torch.nn.functional.softplus(dl - 1.0)
    A = -torch.exp(torch.rand(D, N, generator=g, dtype=dtype) * math.log(16.0))
    shape = (B, N, L) if G == 1 else (B, G, N, L)
    Bm = torch.randn(*shape, generator=g, dtype=dtype)
    Cm = torch.randn(*shape, generator=g, dtype=dtype)
    Dv = torch.randn(D, generator=g, dtype=dtype)
    zz = torch.randn(B, D, L, generator=g, dtype=dtype) if z else None
    bb = torch.randn(D, generator=g, dtype=dtype) * 0.3 if bias else None
    return u, dl, A, Bm, Cm, Dv, zz, bb


def _np(t):
    return None if t is None else t.detach().double().numpy()


CASES = [
    dict(),
    dict(G=2, D=8),
    dict(G=3, D=6, z=True),
    dict(z=True, bias=True),
    dict(N=1),
    dict(L=1),
    dict(B=1, D=3, L=40, N=7, G=1, z=True, bias=True),
]


@pytest.mark.parametrize("kw", CASES)
def test_restatement_forward_matches_brute64(kw):
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(**kw)
    sp = b is not None
    out, ls = selective_scan_ref(u, dl, A, Bm, Cm, Dv, z, b, sp, True, compute_dtype=F64)
    f = scan_fwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(Dv), _np(z), _np(b), sp)
    np.testing.assert_allclose(out.numpy(), f["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ls.numpy(), f["last_state"], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("kw", CASES)
def test_restatement_gradients_match_hand_derived_backward(kw):
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(**kw, seed=3)
    sp = b is not None
    dout = torch.randn_like(u)
    g = selective_scan_ref_grads(u, dl, A, Bm, Cm, Dv, dout, z=z, delta_bias=b,
                                 delta_softplus=sp, compute_dtype=F64)
    h = scan_bwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(dout), _np(Dv), _np(z),
                   _np(b), sp)
    for k in ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias"):
        if g[k] is None:
            assert h[k] is None
            continue
        np.testing.assert_allclose(g[k].numpy(), h[k], rtol=1e-10, atol=1e-10, err_msg=k)


def test_gradcheck_restatement():
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(B=1, D=3, L=5, N=2, G=1, z=True, bias=True, seed=5)
    fn = lambda *a: selective_scan_ref(*a, delta_softplus=True, compute_dtype=F64)
    ins = tuple(t.clone().requires_grad_() for t in (u, dl, A, Bm, Cm, Dv, z, b))
    assert torch.autograd.gradcheck(fn, ins, eps=1e-6, atol=1e-7, rtol=1e-6)


def test_varlen_matches_brute64_resets():
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(B=1, D=5, L=30, N=3, z=True, bias=True, seed=7)
    cu = torch.tensor([0, 4, 5, 5, 21, 30], dtype=torch.int32)
    out, ls = selective_scan_ref_varlen(u, dl, A, Bm, Cm, cu, Dv, z, b, True, True,
                                        compute_dtype=F64)
    f = scan_fwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(Dv), _np(z), _np(b), True,
                   cu_seqlens=cu.numpy())
    np.testing.assert_allclose(out.numpy(), f["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ls.numpy(), f["last_state"], rtol=1e-12, atol=1e-12)
    assert not ls[2].any()  # sequence 2 is empty
    dout = torch.randn_like(u)
    cu2 = torch.tensor([0, 4, 5, 21, 30], dtype=torch.int32)
    g = selective_scan_ref_grads(u, dl, A, Bm, Cm, Dv, dout, z=z, delta_bias=b, delta_softplus=True,
                                 cu_seqlens=cu2, compute_dtype=F64)
    h = scan_bwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(dout), _np(Dv), _np(z), _np(b),
                   True, cu_seqlens=cu2.numpy())
    for k in ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias"):
        np.testing.assert_allclose(g[k].numpy(), h[k], rtol=1e-10, atol=1e-10, err_msg=k)


# ---------------------------------------------------------------- closed forms

def test_closed_form_single_step():
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(L=1, seed=11)
    out = selective_scan_ref(u, dl, A, Bm, Cm, Dv, compute_dtype=F64)
    want = dl * u * (Bm * Cm).sum(1, keepdim=True) + Dv[None, :, None] * u
    torch.testing.assert_close(out, want, rtol=1e-12, atol=1e-12)


def test_closed_form_geometric_series():
    B, D, L, N = 1, 3, 50, 4
    delta = torch.full((B, D, L), 0.3, dtype=F64)
    A = -torch.tensor([[0.5, 1.0, 2.0, 4.0]] * D, dtype=F64)
    ones = torch.ones(B, N, L, dtype=F64)
    u = torch.ones(B, D, L, dtype=F64)
    out, ls = selective_scan_ref(u, delta, A, ones, ones, return_last_state=True, compute_dtype=F64)
    a = torch.exp(0.3 * A[0])                           # [N]
    t = torch.arange(L, dtype=F64)[:, None]
    h = 0.3 * (1 - a ** (t + 1)) / (1 - a)              # [L, N]
    torch.testing.assert_close(out[0, 0], h.sum(1), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ls[0, 0], h[-1], rtol=1e-12, atol=1e-12)


def test_closed_form_zero_delta_is_skip_only():
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(L=12, seed=12)
    out, ls = selective_scan_ref(u, torch.zeros_like(dl), A, Bm, Cm, Dv, return_last_state=True,
                                 compute_dtype=F64)
    torch.testing.assert_close(out, u * Dv[None, :, None], rtol=0, atol=0)
    assert torch.count_nonzero(ls) == 0


def test_closed_form_no_memory():
    # abar = exp(Delta A) underflows to 0: h_t = Delta_t u_t B_t
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(L=10, seed=13)
    dl = dl + 0.5
    A = torch.full_like(A, -1e4)
    out = selective_scan_ref(u, dl, A, Bm, Cm, Dv, compute_dtype=F64)
    want = dl * u * (Bm * Cm).sum(1)[:, None, :] + Dv[None, :, None] * u
    torch.testing.assert_close(out, want, rtol=1e-12, atol=1e-12)


def test_closed_form_scalar_state():
    u, dl, A, Bm, Cm, _, _, _ = _inputs(B=1, D=1, L=25, N=1, seed=14)
    out = selective_scan_ref(u, dl, A, Bm, Cm, compute_dtype=F64)
    h, ys = 0.0, []
    for t in range(25):
        h = math.exp(dl[0, 0, t].item() * A[0, 0].item()) * h + dl[0, 0, t].item() * u[0, 0, t].item() * Bm[0, 0, t].item()
        ys.append(h * Cm[0, 0, t].item())
    torch.testing.assert_close(out[0, 0], torch.tensor(ys, dtype=F64), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- invariants

def test_causality_prefix():
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(L=40, z=True, bias=True, seed=21)
    full = selective_scan_ref(u, dl, A, Bm, Cm, Dv, z, b, True, compute_dtype=F64)
    pre = selective_scan_ref(u[..., :17], dl[..., :17], A, Bm[..., :17], Cm[..., :17], Dv,
                             z[..., :17], b, True, compute_dtype=F64)
    torch.testing.assert_close(full[..., :17], pre, rtol=0, atol=0)


def test_linearity_in_u():
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(L=30, seed=22)
    u2 = torch.randn_like(u)
    f = lambda x: selective_scan_ref(x, dl, A, Bm, Cm, Dv, compute_dtype=F64)
    torch.testing.assert_close(f(2.5 * u - 1.5 * u2), 2.5 * f(u) - 1.5 * f(u2), rtol=1e-10, atol=1e-10)


def test_chunk_split_state_passing():
    # scan(x[0:L]) restricted to [L1, L) == scan(x[L1:L]) from zero + C_t (prod abar) h_{L1-1}
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(B=2, D=4, L=48, N=5, seed=23)
    L1 = 19
    full = selective_scan_ref(u, dl, A, Bm, Cm, Dv, compute_dtype=F64)
    _, h0 = selective_scan_ref(u[..., :L1], dl[..., :L1], A, Bm[..., :L1], Cm[..., :L1],
                               return_last_state=True, compute_dtype=F64)
    tail = selective_scan_ref(u[..., L1:], dl[..., L1:], A, Bm[..., L1:], Cm[..., L1:], Dv,
                              compute_dtype=F64)
    cum = torch.cumsum(dl[..., L1:], -1)                           # [B, D, L-L1]
    decay = torch.exp(cum[..., None] * A[None, :, None, :])       # [B, D, L-L1, N]
    carry = torch.einsum('bdln,bdn,bnl->bdl', decay, h0, Cm[..., L1:])
    torch.testing.assert_close(full[..., L1:], tail + carry, rtol=1e-10, atol=1e-10)


def test_group_broadcast_equals_repeated_groups():
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(D=8, G=2, seed=24)
    out2 = selective_scan_ref(u, dl, A, Bm, Cm, Dv, compute_dtype=F64)
    out4 = selective_scan_ref(u, dl, A, Bm.repeat_interleave(2, 1), Cm.repeat_interleave(2, 1), Dv,
                              compute_dtype=F64)
    torch.testing.assert_close(out2, out4, rtol=0, atol=0)
    # the first D/G channels read group 0 only
    Bz = Bm.clone()
    Bz[:, 1] = 0
    out_z = selective_scan_ref(u, dl, A, Bz, Cm, Dv, compute_dtype=F64)
    torch.testing.assert_close(out_z[:, :4], out2[:, :4], rtol=0, atol=0)


def test_channel_last_view_is_layout_invariant():
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(L=20, seed=25, dtype=torch.float32)
    a = selective_scan_ref(u, dl, A, Bm, Cm, Dv)
    b = selective_scan_ref(u.mT.contiguous().mT, dl.mT.contiguous().mT, A, Bm.mT.contiguous().mT,
                           Cm.mT.contiguous().mT, Dv)
    torch.testing.assert_close(a, b, rtol=0, atol=0)


def test_softplus_threshold_20():
    u, dl, A, Bm, Cm, Dv, _, _ = _inputs(B=1, D=2, L=4, seed=26)
    big = torch.full_like(dl, 25.0)
    a = selective_scan_ref(u, big, A, Bm, Cm, Dv, delta_softplus=True, compute_dtype=F64)
    b = selective_scan_ref(u, big, A, Bm, Cm, Dv, delta_softplus=False, compute_dtype=F64)
    torch.testing.assert_close(a, b, rtol=0, atol=0)


# ---------------------------------------------------------------- C restatement

@pytest.mark.parametrize("kw", CASES)
def test_c_oracle_forward_matches_restatement(kw):
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(**kw, dtype=torch.float32, seed=31)
    sp = b is not None
    out, ls = selective_scan_ref(u, dl, A, Bm, Cm, Dv, z, b, sp, True)
    co, cls = c_oracle.fwd(u, dl, A, Bm, Cm, Dv, z, b, sp)
    torch.testing.assert_close(co, out, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(cls, ls, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kw", CASES)
def test_c_oracle_backward_matches_brute64(kw):
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(**kw, dtype=torch.float32, seed=32)
    sp = b is not None
    dout = torch.randn_like(u)
    cg = c_oracle.bwd(u, dl, A, Bm, Cm, dout, Dv, z, b, sp)
    h = scan_bwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(dout), _np(Dv), _np(z), _np(b), sp)
    for k in ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias"):
        if h[k] is None:
            continue
        np.testing.assert_allclose(cg[k].numpy(), h[k], rtol=2e-5, atol=2e-5 * np.abs(h[k]).max(),
                                   err_msg=k)


@pytest.mark.parametrize("kw", CASES)
def test_c_oracle_float64_forward_matches_brute64(kw):
    """The C float64 forward (the exact value fp32 results are measured against) equals the
    independent NumPy float64 brute force."""
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(**kw, dtype=torch.float32, seed=34)
    sp = b is not None
    co, cls = c_oracle.fwd64(u, dl, A, Bm, Cm, Dv, z, b, sp)
    h = scan_fwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(Dv), _np(z), _np(b), sp)
    np.testing.assert_allclose(co.numpy(), h["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(cls.numpy(), h["last_state"], rtol=1e-12, atol=1e-12)


def test_c_oracle_varlen():
    u, dl, A, Bm, Cm, Dv, z, b = _inputs(B=1, D=4, L=60, N=6, z=True, bias=True, dtype=torch.float32,
                                         seed=33)
    cu = torch.tensor([0, 1, 30, 31, 60], dtype=torch.int32)
    out, ls = selective_scan_ref_varlen(u, dl, A, Bm, Cm, cu, Dv, z, b, True, True)
    co, cls = c_oracle.fwd(u, dl, A, Bm, Cm, Dv, z, b, True, cu_seqlens=cu)
    torch.testing.assert_close(co, out, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(cls, ls, rtol=1e-5, atol=1e-6)
    dout = torch.randn_like(u)
    co64, cls64 = c_oracle.fwd64(u, dl, A, Bm, Cm, Dv, z, b, True, cu_seqlens=cu)
    h64 = scan_fwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(Dv), _np(z), _np(b), True,
                     cu_seqlens=cu.numpy())
    np.testing.assert_allclose(co64.numpy(), h64["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(cls64.numpy(), h64["last_state"], rtol=1e-12, atol=1e-12)
    cg = c_oracle.bwd(u, dl, A, Bm, Cm, dout, Dv, z, b, True, cu_seqlens=cu)
    h = scan_bwd64(_np(u), _np(dl), _np(A), _np(Bm), _np(Cm), _np(dout), _np(Dv), _np(z), _np(b),
                   True, cu_seqlens=cu.numpy())
    for k in ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias"):
        np.testing.assert_allclose(cg[k].numpy(), h[k], rtol=2e-5, atol=2e-5 * np.abs(h[k]).max(),
                                   err_msg=k)


# ---------------------------------------------------------------- golden fixtures

def _golden_cases():
    with np.load(GOLDEN) as z:
        names = sorted({k.split("/")[0] for k in z.files})
    return names


@pytest.mark.parametrize("name", _golden_cases())
def test_golden_fixtures_reproduced_by_restatement(name):
    with np.load(GOLDEN) as z:
        d = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    t = lambda k: torch.from_numpy(d[k]).double() if k in d else None
    sp = "delta_bias" in d
    if "cu_seqlens" in d:
        out, ls = selective_scan_ref_varlen(t("u"), t("delta"), t("A"), t("B"), t("C"),
                                            torch.from_numpy(d["cu_seqlens"]), t("D"), t("z"),
                                            t("delta_bias"), sp, True, compute_dtype=F64)
    else:
        out, ls = selective_scan_ref(t("u"), t("delta"), t("A"), t("B"), t("C"), t("D"), t("z"),
                                     t("delta_bias"), sp, True, compute_dtype=F64)
    np.testing.assert_allclose(out.numpy(), d["ref_out"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(ls.numpy(), d["ref_last_state"], rtol=1e-11, atol=1e-11)


def test_ssm_mixer_restatement_matches_selective_scan_ref():
    """The SSMMixer loop (backbone.py:1207-1242) and selective_scan_ref (SSI:91-157) are the
    same recurrence in two layouts: with softplus on dt, D skip and z gate they agree to
    float64 rounding."""
    from oracle.ssm_mixer_ref import ssm_mixer_scan_ref
    g = torch.Generator().manual_seed(21)
    B, L, I, N = 2, 40, 24, 8
    f64 = dict(generator=g, dtype=torch.float64)
    x_conv, dt_lin, z = (torch.randn(B, L, I, **f64) for _ in range(3))
    A_log = torch.log(torch.arange(1, N + 1, dtype=torch.float64))[None].repeat(I, 1)
    A_log = A_log + 0.1 * torch.randn(I, N, **f64)
    Bp, Cp = torch.randn(B, L, N, **f64), torch.randn(B, L, N, **f64)
    Dv = torch.randn(I, **f64)
    y1 = ssm_mixer_scan_ref(x_conv, dt_lin, A_log, Bp, Cp, Dv, z)
    y2 = selective_scan_ref(x_conv.mT, dt_lin.mT, -torch.exp(A_log), Bp.mT, Cp.mT, D=Dv, z=z.mT,
                            delta_softplus=True, compute_dtype=torch.float64).mT
    assert torch.allclose(y1, y2, rtol=1e-12, atol=1e-12)
