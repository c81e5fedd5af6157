"""Pins the Mamba-2 SSD restatements (oracle/ssd_ref.py) on the CPU: the chunked restatement
of the reference pipeline equals an independent float64 loop over the recurrence, and that
loop equals the S6 float64 brute force through the head expansion the reference uses to
express SSD as a selective scan (ssd_combined.py:663-711)."""
import numpy as np
import pytest
import torch

from oracle.brute64 import scan_fwd64
from oracle.ssd_ref import ssd_brute64, ssd_chunked_ref


def inputs(batch=2, L=37, H=4, P=3, G=2, N=5, seed=0, D_hdim=False):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    return dict(x=r(batch, L, H, P), dt=0.5 * r(batch, L, H) - 1.0,
                A=-torch.exp(r(H) * 0.5), B=r(batch, L, G, N), C=r(batch, L, G, N),
                D=r(H, P) if D_hdim else r(H), z=r(batch, L, H, P), dt_bias=0.3 * r(H))


def test_brute_force_is_the_selective_scan_of_the_head_expansion():
    t = inputs(D_hdim=True)
    out, final = ssd_brute64(**t, dt_softplus=True)
    b, L, H, P = t["x"].shape
    G, N = t["B"].shape[2:]
    u = t["x"].permute(0, 2, 3, 1).reshape(b, H * P, L)
    delta = t["dt"].permute(0, 2, 1).repeat_interleave(P, dim=1)
    A = t["A"].repeat_interleave(P)[:, None].expand(H * P, N)
    Bm, Cm = t["B"].permute(0, 2, 3, 1), t["C"].permute(0, 2, 3, 1)
    want = scan_fwd64(u.numpy(), delta.numpy(), A.numpy(), Bm.numpy(), Cm.numpy(),
                      D=t["D"].reshape(-1).numpy(), z=t["z"].permute(0, 2, 3, 1).reshape(b, H * P, L).numpy(),
                      delta_bias=t["dt_bias"].repeat_interleave(P).numpy(), delta_softplus=True)
    np.testing.assert_allclose(out, want["out"].reshape(b, H, P, L).transpose(0, 3, 1, 2),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(final, want["last_state"].reshape(b, H, P, N), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("chunk", [4, 8, 64])
@pytest.mark.parametrize("opts", ["plain", "full", "init", "seq", "seq_init", "limit", "D_hdim"])
def test_chunked_restatement_matches_brute_force(chunk, opts):
    t = inputs(seed=3, D_hdim=opts == "D_hdim")
    kw = dict(dt_softplus=True)
    if opts == "plain":
        t.pop("z"); t.pop("D"); t.pop("dt_bias"); kw = {}
        t["dt"] = torch.nn.functional.softplus(t["dt"])
    if opts in ("init", "seq_init"):
        t["initial_states"] = torch.randn(2, 4, 3, 5, generator=torch.Generator().manual_seed(9),
                                          dtype=torch.float64)
    if opts in ("seq", "seq_init"):
        seq = torch.zeros(2, 37, dtype=torch.int32)
        seq[0, 9:] = 1; seq[0, 22:] = 2; seq[1, 30:] = 1
        t["seq_idx"] = seq
    if opts == "limit":
        kw["dt_limit"] = (0.2, 0.6)
    out, out_x, final = ssd_chunked_ref(**t, chunk_size=chunk, compute_dtype=torch.float64, **kw)
    want, want_final = ssd_brute64(**t, **kw)
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(final.numpy(), want_final, rtol=1e-10, atol=1e-10)


CU = [0, 9, 16, 27, 45, 46, 61]   # chunk 8: ends on a boundary (16), spans chunks (27, 45), length 1


@pytest.mark.parametrize("with_seq", [True, False])
@pytest.mark.parametrize("init", [False, True])
def test_varlen_states_match_the_brute_force_on_each_prefix(with_seq, init):
    """chunk_state_varlen's states, pinned without its own formula:
    * with seq_idx marking the sequences, each is the brute-force state of that sequence
      run alone (the first one from initial_states);
    * without it, a sequence that starts inside its last chunk still gets only its own rows,
      and one that starts earlier gets the unsegmented state at its end (the carried part
      holds the whole history)."""
    from oracle.ssd_ref import ssd_varlen_states_ref
    t = inputs(batch=1, L=61, seed=11)
    for k in ("z", "D", "C"):
        t.pop(k)
    Q = 8
    seq = torch.zeros(1, 61, dtype=torch.int32)
    for i, (s0, s1) in enumerate(zip(CU[:-1], CU[1:])):
        seq[0, s0:s1] = i
    init_st = (torch.randn(1, 4, 3, 5, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
               if init else None)
    got = ssd_varlen_states_ref(**t, chunk_size=Q, cu_seqlens=torch.tensor(CU),
                                initial_states=init_st, seq_idx=seq if with_seq else None,
                                dt_softplus=True, compute_dtype=torch.float64)
    assert got.shape == (len(CU) - 1, 4, 3, 5)
    Cd = torch.zeros(1, 61, 2, 5, dtype=torch.float64)
    for i, (s0, s1) in enumerate(zip(CU[:-1], CU[1:])):
        sl = lambda v: v[:, s0:s1]
        if with_seq or s0 >= (s1 - 1) // Q * Q:
            first = i == 0
            _, want = ssd_brute64(sl(t["x"]), sl(t["dt"]), t["A"], sl(t["B"]), sl(Cd),
                                  dt_bias=t["dt_bias"], dt_softplus=True,
                                  initial_states=init_st if (first and (with_seq or s0 == 0)) else None)
        else:
            pre = lambda v: v[:, :s1]
            _, want = ssd_brute64(pre(t["x"]), pre(t["dt"]), t["A"], pre(t["B"]), pre(Cd),
                                  dt_bias=t["dt_bias"], dt_softplus=True, initial_states=init_st)
        np.testing.assert_allclose(got[i].numpy(), want[0], rtol=1e-10, atol=1e-10, err_msg=f"seq {i}")
