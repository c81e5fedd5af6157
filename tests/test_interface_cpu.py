"""Host logic of the drop-in interface, without a GPU: argument checks follow the
reference's contract (SelectiveScanFn, selective_scan_interface.py:19-88), the variants the
reference's GPU kernel lacks raise NotImplementedError, and CPU tensors raise instead of
silently running some fallback."""
import pytest
import torch

import s6scan
from s6scan.configs import CONFIGS, make_inputs


def small(dtype=torch.float32, B=2, D=8, L=12, N=4, G=None):
    g = torch.Generator().manual_seed(0)
    u = torch.randn(B, D, L, generator=g).to(dtype)
    dl = torch.rand(B, D, L, generator=g).to(dtype)
    A = -torch.rand(D, N, generator=g)
    shape = (B, N, L) if G is None else (B, G, N, L)
    Bm = torch.randn(*shape, generator=g).to(dtype)
    Cm = torch.randn(*shape, generator=g).to(dtype)
    return u, dl, A, Bm, Cm


def test_cpu_tensors_raise_no_fallback():
    u, dl, A, Bm, Cm = small()
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        s6scan.selective_scan_fn(u, dl, A, Bm, Cm)


def test_complex_A_not_implemented():
    u, dl, A, Bm, Cm = small()
    with pytest.raises(NotImplementedError, match="complex"):
        s6scan.check_inputs(u, dl, torch.complex(A, A), Bm, Cm)


def test_time_invariant_BC_not_implemented():
    u, dl, A, Bm, Cm = small()
    with pytest.raises(NotImplementedError, match="time-invariant"):
        s6scan.check_inputs(u, dl, A, torch.randn(8, 4), Cm)


@pytest.mark.parametrize("mutate,exc,msg", [
    (lambda a: a.update(delta=a["delta"][..., :-1]), ValueError, "delta shape"),
    (lambda a: a.update(delta=a["delta"].double()), TypeError, "delta dtype"),
    (lambda a: a.update(A=a["A"].double()), TypeError, "A must be float32"),
    (lambda a: a.update(A=a["A"][:-1]), ValueError, "A must be"),
    (lambda a: a.update(B=a["B"][:, :-1]), ValueError, "B shape"),
    (lambda a: a.update(C=a["C"].half()), TypeError, "C dtype"),
    (lambda a: a.update(D=torch.ones(8, dtype=torch.float64)), ValueError, "D must be"),
    (lambda a: a.update(z=torch.ones(2, 8, 11)), ValueError, "z shape"),
    (lambda a: a.update(delta_bias=torch.ones(7)), ValueError, "delta_bias"),
])
def test_argument_errors(mutate, exc, msg):
    u, dl, A, Bm, Cm = small()
    a = dict(u=u, delta=dl, A=A, B=Bm, C=Cm)
    mutate(a)
    with pytest.raises(exc, match=msg):
        s6scan.check_inputs(a["u"], a["delta"], a["A"], a["B"], a["C"], a.get("D"), a.get("z"),
                            a.get("delta_bias"))


def test_groups_and_varlen_checks():
    u, dl, A, Bm, Cm = small(G=3, D=8)
    with pytest.raises(ValueError, match="divisible"):
        s6scan.check_inputs(u, dl, A, Bm, Cm)
    u, dl, A, Bm, Cm = small()
    with pytest.raises(ValueError, match="batch == 1"):
        s6scan.check_inputs(u, dl, A, Bm, Cm, cu_seqlens=torch.tensor([0, 12], dtype=torch.int32))
    u, dl, A, Bm, Cm = small(B=1)
    with pytest.raises(ValueError, match="int32"):
        s6scan.check_inputs(u, dl, A, Bm, Cm, cu_seqlens=torch.tensor([0, 12]))


def test_dstate_limit():
    u, dl, A, Bm, Cm = small(N=65)
    with pytest.raises(NotImplementedError, match="dstate"):
        s6scan.check_inputs(u, dl, A, Bm, Cm)


def test_workload_generators_match_declared_shapes():
    for k in (0, 1):
        cfg = CONFIGS[k]
        x = make_inputs(cfg, seqlen=64, batch=1)
        assert x["x"].shape == (1, 64, cfg.dim) and x["x"].dtype == cfg.dtype
        assert x["A"].dtype == torch.float32 and (x["A"] < 0).all()
        assert (x["delta"].float() > 0).all()
    v = make_inputs(CONFIGS[4], seqlen=4096, dim=64)
    cu = v["cu_seqlens"]
    assert cu.dtype == torch.int32 and cu[0] == 0 and cu.numel() == 65
    assert int(cu[-1]) == v["x"].shape[1]
    assert CONFIGS[1].algorithmic_bytes() == 210256896
    assert CONFIGS[0].algorithmic_bytes() == 1720832


@pytest.mark.parametrize("cu,msg", [
    ([10, 100], r"cu_seqlens\[0\] must be 0"),
    ([0, 60, 50, 100], "non-decreasing"),
    ([0, 50], "must equal seqlen 100"),
])
def test_malformed_cu_seqlens_rejected_before_launch(cu, msg):
    """check_inputs reads the offsets once and rejects a vector that does not start at 0, is
    not non-decreasing or does not end at seqlen (ssd_combined.py:576-577,
    ssd_state_passing.py:76-78): such a vector never reaches a kernel."""
    u, dl, A, Bm, Cm = small(B=1, L=100)
    with pytest.raises(ValueError, match=msg):
        s6scan.check_inputs(u, dl, A, Bm, Cm, cu_seqlens=torch.tensor(cu, dtype=torch.int32))
    # the public entry point raises the same error (before any device check)
    with pytest.raises(ValueError, match=msg):
        s6scan.selective_scan_fn(u, dl, A, Bm, Cm, cu_seqlens=torch.tensor(cu, dtype=torch.int32))


def test_wellformed_cu_seqlens_accepted():
    # the offsets pass; the only remaining complaint is the CPU device (no fallback)
    u, dl, A, Bm, Cm = small(B=1, L=100)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        s6scan.check_inputs(u, dl, A, Bm, Cm,
                            cu_seqlens=torch.tensor([0, 30, 30, 100], dtype=torch.int32))


def test_legacy_conv_module_signatures():
    """s6scan.causal_conv1d_legacy has the argument lists of the conv module calls in the
    interface file zoology's Mamba imports (mamba_ssm/selective_scan_interface.py:181,
    288-290, 321); s6scan.causal_conv1d those of the ops copy (ops/...:187-189, 299-301)."""
    import inspect

    from s6scan import causal_conv1d as new
    from s6scan import causal_conv1d_legacy as old

    def names(f):
        return list(inspect.signature(f).parameters)

    assert names(old.causal_conv1d_fwd) == ["x", "weight", "bias", "seq_idx", "silu_activation"]
    assert names(old.causal_conv1d_bwd) == ["x", "weight", "bias", "dout", "seq_idx", "dx",
                                            "silu_activation"]
    assert len(names(new.causal_conv1d_fwd)) == 7 and len(names(new.causal_conv1d_bwd)) == 10
    # a CPU tensor still raises (no fallback) through either arity
    x = torch.randn(1, 4, 8)
    with pytest.raises(RuntimeError, match="ROCm"):
        old.causal_conv1d_fwd(x, torch.randn(4, 3), None, None, True)
    with pytest.raises(RuntimeError, match="ROCm"):
        old.causal_conv1d_fn(x, torch.randn(4, 3), None, "silu")
