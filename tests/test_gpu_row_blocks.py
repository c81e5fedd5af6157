"""The chunked forward's two access forms.  For u / delta / z / out / out_z with a contiguous
time axis (the [B, D, L] layout of the reference's callers, mamba.py:128-132) and seqlen a
multiple of 8, each lane moves whole 8-step row blocks with 16-byte accesses; otherwise one
step at a time.  The arithmetic is the same, so out, out_z, the checkpoints and the final
states must be bit-identical between the two (S6_FWD_ROWVEC=0 forces per-step accesses on the
same tensors), and ``forward_kernel`` must name the form that ran (the single-pass kernel, which
L-contiguous inputs otherwise get at these dstates, is switched off with S6_FWD_PATH=chunked).  The per-step form is
held to the oracle by the parity tests; the row-block form is too, by the contiguous-layout
cases there."""
import pytest
import torch

from s6scan.selective_scan_interface import forward_kernel, selective_scan_forward
from test_gpu_parity import bc_views, gen, views

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # B, L, D, N, dtype, z, bias, cu_seqlens
    (2, 1024, 128, 16, torch.bfloat16, False, False, None),
    (2, 1000, 96, 16, torch.float32, True, True, None),
    (1, 2048, 200, 8, torch.float16, True, False, None),
    (2, 512, 64, 32, torch.bfloat16, False, True, None),
    (3, 4096, 256, 16, torch.bfloat16, True, True, None),
    (2, 776, 64, 24, torch.float32, False, False, None),
    (1, 3000, 128, 16, torch.bfloat16, False, False, [0, 3, 700, 701, 2999, 3000]),
    (1, 2400, 64, 16, torch.float32, True, True, [0, 8, 16, 1000, 2400]),
]


def _run(inp, cu):
    x, dl = views(inp["x"].to(DEV), "contiguous"), views(inp["delta"].to(DEV), "contiguous")
    z = views(inp["z"].to(DEV), "contiguous") if inp["z"] is not None else None
    Bm, Cm = bc_views(inp["B"].to(DEV), 1, "contiguous"), bc_views(inp["C"].to(DEV), 1, "contiguous")
    A, D = inp["A"].to(DEV), inp["D"].to(DEV)
    bias = inp["bias"].to(DEV) if inp["bias"] is not None else None
    cu = torch.tensor(cu, dtype=torch.int32, device=DEV) if cu is not None else None
    kw = dict(D=D, z=z, delta_bias=bias, delta_softplus=inp["softplus"], cu_seqlens=cu)
    rows = forward_kernel(x, dl, A, Bm, Cm, **kw) == "chunked_rows"
    res = selective_scan_forward(x, dl, A, Bm, Cm, **kw, want_ckpt=True, want_last_state=True)
    torch.cuda.synchronize()
    return rows, res


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c[:7])).replace("torch.", ""))
def test_row_blocks_bit_identical_to_per_step(case, monkeypatch):
    B, L, D, N, dtype, z, bias, cu = case
    inp = gen(B, L, D, N, dtype, seed=L + N, z=z, bias=bias)
    monkeypatch.setenv("S6_FWD_PATH", "chunked")
    monkeypatch.delenv("S6_FWD_ROWVEC", raising=False)
    print(f"case {case}: row blocks", flush=True)
    rows, got = _run(inp, cu)
    assert rows, "expected the row-block form for this layout"
    monkeypatch.setenv("S6_FWD_ROWVEC", "0")
    print(f"case {case}: per step", flush=True)
    rows0, ref = _run(inp, cu)
    assert not rows0
    for name, a, b in zip(("out", "out_z", "x_ckpt", "last_state"), got, ref):
        if b is None:
            assert a is None
            continue
        assert torch.equal(a, b), f"{name}: max |diff| {(a.float() - b.float()).abs().max().item():.3g}"


def test_channel_last_and_unaligned_take_per_step_form(monkeypatch):
    """The bench's channel-last views and an L-contiguous layout whose rows are not 16-byte
    aligned take the per-step form (no device work: a host query)."""
    monkeypatch.setenv("S6_FWD_PATH", "chunked")
    monkeypatch.delenv("S6_FWD_ROWVEC", raising=False)
    inp = gen(2, 1024, 128, 16, torch.bfloat16, seed=3)
    A, D = inp["A"].to(DEV), inp["D"].to(DEV)
    Bm, Cm = bc_views(inp["B"].to(DEV), 1, "view"), bc_views(inp["C"].to(DEV), 1, "view")
    x, dl = views(inp["x"].to(DEV), "view"), views(inp["delta"].to(DEV), "view")
    assert forward_kernel(x, dl, A, Bm, Cm, D=D) == "chunked"
    xc = views(inp["x"].to(DEV), "contiguous")
    assert forward_kernel(xc, xc, A, Bm, Cm, D=D) == "chunked_rows"
    big = torch.empty(2, 128, 1028, dtype=torch.bfloat16, device=DEV)
    xs = big[:, :, 2:1026]                         # rows start 4 bytes past 16-byte alignment
    assert forward_kernel(xs, xc, A, Bm, Cm, D=D) == "chunked"


BWD_CASES = [
    # B, L, D, N, dtype, z, bias, cu_seqlens, recompute_out_z
    (2, 1024, 128, 16, torch.bfloat16, False, False, None, False),
    (2, 1000, 96, 16, torch.float32, True, True, None, False),
    (1, 2048, 200, 8, torch.float16, True, False, None, True),
    (2, 512, 64, 16, torch.bfloat16, True, True, None, True),
    (2, 4096, 192, 16, torch.bfloat16, False, True, None, False),
    (1, 3000, 128, 16, torch.bfloat16, False, True, [0, 3, 700, 701, 2999, 3000], False),
]


@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: "-".join(map(str, c[:7])).replace("torch.", ""))
def test_backward_row_blocks_bit_identical_to_per_step(case, monkeypatch):
    """The backward on L-contiguous tensors: row blocks against per-step accesses
    (S6_BWD_ROWVEC=0) on the same forward outputs, every gradient bit for bit."""
    from s6scan.selective_scan_interface import backward_row_blocks, selective_scan_backward

    B, L, D, N, dtype, z, bias, cu, oz = case
    inp = gen(B, L, D, N, dtype, seed=L + 2 * N, z=z, bias=bias)
    monkeypatch.delenv("S6_BWD_ROWVEC", raising=False)
    lc = lambda t: views(t.to(DEV), "contiguous") if t is not None else None
    x, dl, zz, dy = lc(inp["x"]), lc(inp["delta"]), lc(inp["z"]), lc(inp["dy"])
    Bm, Cm = bc_views(inp["B"].to(DEV), 1, "contiguous"), bc_views(inp["C"].to(DEV), 1, "contiguous")
    A, Dv = inp["A"].to(DEV), inp["D"].to(DEV)
    bb = inp["bias"].to(DEV) if inp["bias"] is not None else None
    cu = torch.tensor(cu, dtype=torch.int32, device=DEV) if cu is not None else None
    sp = inp["softplus"]
    out, _, xck, _ = selective_scan_forward(x, dl, A, Bm, Cm, D=Dv, z=zz, delta_bias=bb,
                                            delta_softplus=sp, cu_seqlens=cu, want_ckpt=True)
    bwd = lambda: selective_scan_backward(x, dl, A, Bm, Cm, Dv, zz, bb, sp, dy, xck,
                                          out=out if z else None, cu_seqlens=cu,
                                          recompute_out_z=oz)
    q = lambda: backward_row_blocks(x, dl, A, Bm, Cm, Dv, zz, bb, sp, dy,
                                    out=out if z else None, cu_seqlens=cu, recompute_out_z=oz)
    assert q(), "expected the row-block backward for this layout"
    print(f"case {case}: row blocks", flush=True)
    got = bwd()
    torch.cuda.synchronize()
    monkeypatch.setenv("S6_BWD_ROWVEC", "0")
    assert not q()
    print(f"case {case}: per step", flush=True)
    ref = bwd()
    torch.cuda.synchronize()
    names = ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias", "out_z")
    assert len(got) == len(ref)
    for name, a, b in zip(names, got, ref):
        if b is None:
            assert a is None, name
            continue
        assert torch.equal(a, b), f"{name}: max |diff| {(a.float() - b.float()).abs().max().item():.3g}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chunked_row_blocks_match_restatement(dtype, monkeypatch):
    """The chunked row-block forward (forced: L-contiguous inputs at dstate 16 otherwise take
    the single-pass kernel) against the oracle, z gate and softplus bias included; fp32 against
    the float64 evaluation of the restatement (see test_forward_matches_restatement)."""
    from test_gpu_parity import ref_fwd, ref_fwd64
    from tolerances import assert_out_close, assert_state_close

    monkeypatch.setenv("S6_FWD_PATH", "chunked")
    monkeypatch.delenv("S6_FWD_ROWVEC", raising=False)
    inp = gen(2, 1000, 128, 16, dtype, seed=21, z=True, bias=True)
    rows, (out, out_z, _, ls) = _run(inp, None)
    assert rows
    ref, ref_ls = ref_fwd64(inp) if dtype == torch.float32 else ref_fwd(inp)
    assert_out_close(out_z, ref, dtype, dstate=16)
    assert_state_close(ls, ref_ls)
