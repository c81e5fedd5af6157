"""Pins the causal conv1d and fused-Mamba restatements (oracle/mamba_inner_ref.py) on the CPU:
against a float64 loop of the defining sum, the impulse response, the width-2 identity,
causality, a hand-derived backward, and a float64 NumPy composition of the whole block."""
import numpy as np
import pytest
import torch

from oracle.brute64 import scan_fwd64
from oracle.mamba_inner_ref import causal_conv1d_loop64, causal_conv1d_ref, mamba_inner_ref


def _rand(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


@pytest.mark.parametrize("width", [2, 3, 4])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("act", [None, "silu"])
def test_conv_ref_matches_float64_loop(width, bias, act):
    x = _rand(2, 5, 11, seed=1)
    w = _rand(5, width, seed=2)
    b = _rand(5, seed=3) if bias else None
    got = causal_conv1d_ref(x, w, b, activation=act).numpy()
    want = causal_conv1d_loop64(x.numpy(), w.numpy(), None if b is None else b.numpy(),
                                silu=act == "silu")
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("width", [2, 3, 4])
def test_conv_impulse_response_is_the_reversed_kernel(width):
    L, s = 12, 4
    x = torch.zeros(1, 3, L, dtype=torch.float64)
    x[:, :, s] = 1.0
    w = _rand(3, width, seed=4)
    b = _rand(3, seed=5)
    out = causal_conv1d_ref(x, w, b)
    want = b[None, :, None].expand(1, 3, L).clone()
    for j in range(width):
        want[:, :, s + j] += w[:, width - 1 - j]
    torch.testing.assert_close(out, want, rtol=0, atol=1e-15)


def test_conv_width2_identity():
    x = _rand(2, 4, 9, seed=6)
    w = torch.tensor([[0.0, 1.0]], dtype=torch.float64).repeat(4, 1)
    b = _rand(4, seed=7)
    torch.testing.assert_close(causal_conv1d_ref(x, w, b), x + b[None, :, None])


def test_conv_is_causal():
    x = _rand(1, 3, 16, seed=8)
    w, b = _rand(3, 4, seed=9), _rand(3, seed=10)
    y = causal_conv1d_ref(x, w, b, activation="silu")
    x2 = x.clone()
    x2[..., 10:] = _rand(1, 3, 6, seed=11)
    y2 = causal_conv1d_ref(x2, w, b, activation="silu")
    torch.testing.assert_close(y[..., :10], y2[..., :10], rtol=0, atol=0)
    assert not torch.allclose(y[..., 10:], y2[..., 10:])


def conv_bwd_loop64(x, w, b, dout, silu):
    """The backward the HIP kernel implements, by hand in float64:
    dpre_t = dout_t act'(pre_t);  dx_s = sum_k w_k dpre_{s+W-1-k};
    dw_k = sum_t dpre_t x_{t-W+1+k};  dbias = sum_t dpre_t."""
    batch, dim, L = x.shape
    W = w.shape[1]
    pre = causal_conv1d_loop64(x, w, b, silu=False)
    sg = 1.0 / (1.0 + np.exp(-pre))
    dpre = dout * (sg * (1.0 + pre * (1.0 - sg)) if silu else 1.0)
    dx = np.zeros_like(x)
    dw = np.zeros_like(w)
    for s in range(L):
        for k in range(W):
            t = s + W - 1 - k
            if t < L:
                dx[:, :, s] += w[None, :, k] * dpre[:, :, t]
    for t in range(L):
        for k in range(W):
            s = t - W + 1 + k
            if s >= 0:
                dw[:, k] += (dpre[:, :, t] * x[:, :, s]).sum(0)
    return dx, dw, dpre.sum(axis=(0, 2))


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("L", [1, 3, 13])
def test_conv_hand_backward_matches_autograd(silu, L):
    x = _rand(2, 4, L, seed=12).requires_grad_(True)
    w = _rand(4, 4, seed=13).requires_grad_(True)
    b = _rand(4, seed=14).requires_grad_(True)
    dout = _rand(2, 4, L, seed=15)
    y = causal_conv1d_ref(x, w, b, activation="silu" if silu else None)
    gx, gw, gb = torch.autograd.grad((y * dout).sum(), (x, w, b))
    dx, dw, db = conv_bwd_loop64(x.detach().numpy(), w.detach().numpy(), b.detach().numpy(),
                                 dout.numpy(), silu)
    np.testing.assert_allclose(gx.numpy(), dx, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gw.numpy(), dw, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gb.numpy(), db, rtol=1e-10, atol=1e-12)


def _block(seed, batch=2, L=7, d_model=6, d_inner=8, d_state=4, dt_rank=3, width=4):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64) * 0.5
    return dict(
        xz=r(batch, 2 * d_inner, L), conv1d_weight=r(d_inner, 1, width), conv1d_bias=r(d_inner),
        x_proj_weight=r(dt_rank + 2 * d_state, d_inner), delta_proj_weight=r(d_inner, dt_rank),
        out_proj_weight=r(d_model, d_inner), out_proj_bias=r(d_model),
        A=-torch.exp(r(d_inner, d_state)), D=r(d_inner), delta_bias=r(d_inner),
        B_proj_bias=r(d_state), C_proj_bias=r(d_state))


def _block_np(p):
    """The fused block composed in float64 NumPy from the two brute forces, with every
    layout change written as explicit index arithmetic."""
    n = {k: (v.numpy() if torch.is_tensor(v) else v) for k, v in p.items()}
    xz = n["xz"]
    batch, two_d, L = xz.shape
    d_inner = two_d // 2
    R = n["delta_proj_weight"].shape[1]
    N = n["A"].shape[1]
    x, z = xz[:, :d_inner], xz[:, d_inner:]
    conv = causal_conv1d_loop64(x, n["conv1d_weight"][:, 0], n["conv1d_bias"], silu=True)
    x_dbl = np.einsum("bdl,kd->blk", conv, n["x_proj_weight"])            # [b, l, R + 2N]
    delta = np.einsum("blr,dr->bdl", x_dbl[:, :, :R], n["delta_proj_weight"])
    B = np.transpose(x_dbl[:, :, R:R + N] + n["B_proj_bias"], (0, 2, 1))  # [b, N, l]
    C = np.transpose(x_dbl[:, :, R + N:] + n["C_proj_bias"], (0, 2, 1))
    f = scan_fwd64(conv, delta, n["A"], B, C, D=n["D"], z=z, delta_bias=n["delta_bias"],
                   delta_softplus=True)
    return np.einsum("bdl,ed->ble", f["out"], n["out_proj_weight"]) + n["out_proj_bias"]


@pytest.mark.parametrize("proj_bias", [False, True])
def test_mamba_inner_ref_matches_float64_composition(proj_bias):
    p = _block(20)
    if not proj_bias:
        p["B_proj_bias"] = p["C_proj_bias"] = None
    got = mamba_inner_ref(**p, delta_softplus=True, compute_dtype=torch.float64).numpy()
    q = dict(p)
    if not proj_bias:
        q["B_proj_bias"] = q["C_proj_bias"] = np.zeros(p["A"].shape[1])
    want = _block_np(q)
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)


def test_mamba_inner_ref_gradcheck():
    p = _block(21, batch=1, L=4, d_model=3, d_inner=4, d_state=2, dt_rank=2, width=3)
    names = ["xz", "conv1d_weight", "x_proj_weight", "delta_proj_weight", "out_proj_weight",
             "A", "D", "B_proj_bias"]
    leaves = [p[k].clone().requires_grad_(True) for k in names]

    def f(*vals):
        q = dict(p)
        q.update(zip(names, vals))
        return mamba_inner_ref(**q, compute_dtype=torch.float64)

    assert torch.autograd.gradcheck(f, leaves, eps=1e-6, atol=1e-6)
