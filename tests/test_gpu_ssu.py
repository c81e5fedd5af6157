"""GPU parity of selective_state_update (s6scan.selective_state_update) against the CPU
restatement (oracle/selective_state_update_ref.py, selective_state_update.py:204-265), and
against the HIP scan itself: a run of decode steps must reproduce selective_scan_fn."""
import pytest
import torch

import s6scan  # noqa: F401
from oracle.selective_state_update_ref import selective_state_update_ref
from s6scan import selective_scan_fn
from s6scan.selective_state_update import selective_state_update
from tolerances import assert_close, assert_out_close, rms

pytestmark = pytest.mark.gpu
DEV = "cuda"


def inputs(batch, nheads, dim, dstate, ngroups, io, st_dtype, bc, seed, heads=True, full=True,
           softplus=True):
    """dt is a raw pre-softplus value, or (softplus False) an already positive step, as
    callers pass it: a negative step would make exp(A dt) > 1 and the state explode."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    hs = (batch, nheads, dim) if heads else (batch, dim)
    dt = 0.5 * r(*hs) - 1.0
    t = dict(
        state=r(batch, nheads, dim, dstate).to(st_dtype) if heads else r(batch, dim, dstate).to(st_dtype),
        x=r(*hs).to(io), dt=(dt if softplus else torch.nn.functional.softplus(dt)).to(io),
        A=-torch.exp(r(nheads, dim, dstate)) if heads else -torch.exp(r(dim, dstate)),
        B=r(batch, ngroups, dstate).to(bc) if heads else r(batch, dstate).to(bc),
        C=r(batch, ngroups, dstate).to(bc) if heads else r(batch, dstate).to(bc))
    if full:
        t.update(D=r(nheads, dim) if heads else r(dim), z=r(*hs).to(io),
                 dt_bias=0.3 * r(nheads, dim) if heads else 0.3 * r(dim))
    return t


def run_both(t, softplus):
    gpu = {k: v.to(DEV) for k, v in t.items()}
    cpu = {k: v.clone() for k, v in t.items()}
    out = selective_state_update(**gpu, dt_softplus=softplus)
    ref = selective_state_update_ref(**{k: (v.float() if k not in ("state",) else v)
                                        for k, v in cpu.items()}, dt_softplus=softplus)
    return out, gpu["state"], ref, cpu["state"]


CASES = [  # batch, nheads, dim, dstate, ngroups, io, state, bc, heads
    (3, 1, 200, 16, 1, torch.float32, torch.float32, torch.float32, False),
    (2, 4, 64, 32, 2, torch.float32, torch.float32, torch.float32, True),
    (2, 4, 64, 32, 4, torch.bfloat16, torch.float32, torch.bfloat16, True),
    (2, 2, 96, 16, 1, torch.bfloat16, torch.bfloat16, torch.bfloat16, True),
    (1, 3, 70, 12, 3, torch.float16, torch.float16, torch.float32, True),
    (4, 1, 33, 1, 1, torch.float32, torch.float32, torch.float32, False),
    (2, 2, 64, 64, 1, torch.float32, torch.float32, torch.float32, True),
    (1, 2, 40, 256, 2, torch.float32, torch.float32, torch.float32, True),
    (1, 1, 1536, 16, 1, torch.bfloat16, torch.float32, torch.bfloat16, False),
]


@pytest.mark.parametrize("softplus", [True, False])
@pytest.mark.parametrize("case", CASES)
def test_state_update_matches_reference(case, softplus):
    batch, nheads, dim, dstate, ngroups, io, sd, bc, heads = case
    t = inputs(batch, nheads, dim, dstate, ngroups, io, sd, bc, seed=dim + dstate, heads=heads,
               softplus=softplus)
    if not softplus:  # the bias would make the step negative again
        t.pop("dt_bias")
    out, st, ref, st_ref = run_both(t, softplus)
    assert out.shape == t["x"].shape and out.dtype == io
    assert_out_close(out, ref, io, "out", dstate=dstate)
    if sd == torch.float32:
        assert_close(st, st_ref, 1e-5, 1e-6, "state")
    else:  # one rounding of the same fp32 value; allow one 16-bit ulp
        assert_close(st, st_ref, 1e-2, 1e-3 * rms(st_ref), "state")


def test_state_update_without_optional_inputs():
    t = inputs(2, 2, 64, 16, 2, torch.float32, torch.float32, torch.float32, seed=5, full=False,
               softplus=False)
    out, st, ref, st_ref = run_both(t, False)
    assert_out_close(out, ref, torch.float32, "out")
    assert_close(st, st_ref, 1e-5, 1e-6, "state")


def test_state_in_place_in_a_strided_cache():
    """The state is a slice of a larger inference cache (non-contiguous): only that slice
    changes."""
    t = inputs(3, 2, 48, 16, 1, torch.float32, torch.float32, torch.float32, seed=7)
    cache = torch.randn(5, 2, 48, 24, generator=torch.Generator().manual_seed(8))
    cache_g = cache.to(DEV)
    view = cache_g[1:4, :, :, 4:20]
    view.copy_(t["state"].to(DEV))
    gpu = {k: v.to(DEV) for k, v in t.items() if k != "state"}
    out = selective_state_update(view, **gpu, dt_softplus=True)
    cpu_state = t["state"].clone()
    ref = selective_state_update_ref(cpu_state, **{k: v for k, v in t.items() if k != "state"},
                                     dt_softplus=True)
    assert_out_close(out, ref, torch.float32)
    assert_close(view, cpu_state, 1e-5, 1e-6, "state slice")
    untouched = cache.clone()
    untouched[1:4, :, :, 4:20] = cache_g[1:4, :, :, 4:20].cpu()
    torch.testing.assert_close(cache_g.cpu(), untouched, rtol=0, atol=0)


def test_tied_head_dim():
    """The reference's TIE_HDIM form (Mamba-2 decode): A, dt and dt_bias one value per head,
    passed as zero-stride expansions."""
    batch, nheads, dim, dstate = 2, 4, 32, 16
    g = torch.Generator().manual_seed(9)
    Ah = -torch.exp(torch.randn(nheads, generator=g))
    dth = 0.5 * torch.randn(batch, nheads, generator=g)
    bh = 0.2 * torch.randn(nheads, generator=g)
    t = dict(state=torch.randn(batch, nheads, dim, dstate, generator=g),
             x=torch.randn(batch, nheads, dim, generator=g),
             B=torch.randn(batch, 1, dstate, generator=g), C=torch.randn(batch, 1, dstate, generator=g),
             D=torch.randn(nheads, dim, generator=g), z=torch.randn(batch, nheads, dim, generator=g))
    exp3 = lambda v, dev: v.to(dev)[:, None, None].expand(nheads, dim, dstate)
    gpu = {k: v.to(DEV) for k, v in t.items()}
    out = selective_state_update(**gpu, A=exp3(Ah, DEV), dt=dth.to(DEV)[..., None].expand(batch, nheads, dim),
                                 dt_bias=bh.to(DEV)[:, None].expand(nheads, dim), dt_softplus=True)
    cpu = {k: v.clone() for k, v in t.items()}
    ref = selective_state_update_ref(**cpu, A=Ah[:, None, None].expand(nheads, dim, dstate),
                                     dt=dth[..., None].expand(batch, nheads, dim),
                                     dt_bias=bh[:, None].expand(nheads, dim), dt_softplus=True)
    assert_out_close(out, ref, torch.float32)
    assert_close(gpu["state"], cpu["state"], 1e-5, 1e-6, "state")


def test_decode_steps_continue_the_hip_scan():
    """Prefill L0 steps with selective_scan_fn (return_last_state), then decode the next
    steps one at a time: outputs and final state equal one selective_scan_fn over all
    L0 + L1 steps."""
    batch, dim, dstate, L0, L1 = 2, 128, 16, 300, 20
    g = torch.Generator().manual_seed(11)
    u = torch.randn(batch, dim, L0 + L1, generator=g)
    dl = 0.5 * torch.randn(batch, dim, L0 + L1, generator=g) - 1.0
    A = -torch.exp(torch.randn(dim, dstate, generator=g))
    B = torch.randn(batch, dstate, L0 + L1, generator=g)
    C = torch.randn(batch, dstate, L0 + L1, generator=g)
    D = torch.randn(dim, generator=g)
    z = torch.randn(batch, dim, L0 + L1, generator=g)
    bias = 0.2 * torch.randn(dim, generator=g)
    dv = lambda t: t.to(DEV)
    full, last = selective_scan_fn(dv(u), dv(dl), dv(A), dv(B), dv(C), dv(D), dv(z), dv(bias),
                                   True, True)
    pre, state = selective_scan_fn(dv(u[..., :L0]), dv(dl[..., :L0]), dv(A), dv(B[..., :L0]),
                                   dv(C[..., :L0]), dv(D), dv(z[..., :L0]), dv(bias), True, True)
    outs = []
    for t in range(L0, L0 + L1):
        outs.append(selective_state_update(state, dv(u[..., t]), dv(dl[..., t]), dv(A),
                                           dv(B[..., t]), dv(C[..., t]), D=dv(D), z=dv(z[..., t]),
                                           dt_bias=dv(bias), dt_softplus=True))
    assert_out_close(torch.stack(outs, -1), full[..., L0:], torch.float32, "decoded out")
    assert_close(state, last, 1e-5, 1e-6, "final state")


def test_decode_step_replays_in_a_hip_graph():
    """A decode loop captures the step in a HIP graph (static input buffers, state updated
    in place by every replay).  Each of several replays, with fresh inputs copied in and
    eager work and synchronisations in between, equals the eager call bit for bit."""
    batch, nheads, dim, dstate = 4, 2, 96, 16
    g = torch.Generator().manual_seed(21)
    r = lambda *s: torch.randn(*s, generator=g).to(DEV)
    state = r(batch, nheads, dim, dstate)
    A = -torch.exp(r(nheads, dim, dstate))
    D, bias = r(nheads, dim), 0.2 * r(nheads, dim)
    xs, dts, zs = r(batch, nheads, dim), r(batch, nheads, dim), r(batch, nheads, dim)
    Bs, Cs = r(batch, 1, dstate), r(batch, 1, dstate)
    eager_state = state.clone()
    warm = state.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        selective_state_update(warm, xs, dts, A, Bs, Cs, D, zs, bias, True)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = selective_state_update(state, xs, dts, A, Bs, Cs, D, zs, bias, True)
    for it in range(3):
        for t in (xs, dts, zs, Bs, Cs):
            t.copy_(torch.randn(t.shape, generator=g).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        want = selective_state_update(eager_state, xs, dts, A, Bs, Cs, D, zs, bias, True)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {it}: out"
        assert torch.equal(state, eager_state), f"replay {it}: state"
