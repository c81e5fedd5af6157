"""GPU parity at the edges the seeded workloads do not reach.

* The kernels' softplus (threshold 20, selective_scan_interface.py:111-112) swept over
  delta + bias in [-30, 25], dense around the switch at 20, forward value and gradient, at
  seqlen 1 where the scan output is Delta itself.
* Config 2 (fp32, dstate 64, slow decay): the kernel's distance from the exact (float64)
  value against the fp32 reference restatement's distance, elementwise, on full-length batch
  rows.  This is the measured fact behind the dstate-scaled absolute term of the fp32 bar.
"""
import pytest
import torch

import s6scan
from oracle import c_oracle
from oracle.selective_scan_ref import selective_scan_ref
from s6scan.configs import CONFIGS, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ulp32(v):
    """Spacing of float32 numbers at |v| (float32 tensor in, float32 tensor out)."""
    a = v.abs()
    return torch.nextafter(a, torch.full_like(a, float("inf"))) - a


def _sweep_values():
    coarse = torch.linspace(-30.0, 25.0, 22001)
    dense = torch.linspace(19.9, 20.1, 4001)
    at20 = torch.tensor([20.0])
    around = torch.cat([torch.nextafter(at20, at20 - 1), at20, torch.nextafter(at20, at20 + 1)])
    special = torch.tensor([0.0, -0.0, 1e-8, -1e-8, -17.0, -16.5, 88.0, -88.0])
    return torch.cat([coarse, dense, around, special]).to(torch.float32)


@pytest.mark.parametrize("with_bias", [False, True])
def test_softplus_sweep_forward_and_gradient(with_bias):
    """seqlen 1, dstate 1, u = B = C = 1: out = Delta = softplus(delta + bias) and
    ddelta = softplus'(delta + bias) exactly in the recurrence, so the kernel's softplus and
    its derivative are compared value by value with torch's fp32 F.softplus (threshold 20)
    through the oracle restatement, within 4 float32 ulp.  A value below the smallest normal
    float32 (softplus(x) < 1.18e-38, x < -87.3) may come out flushed to zero, as the GPU's
    fp32 exponential flushes subnormal results; the sweep includes x = -88 to show that this
    is the only effect there."""
    x = _sweep_values()
    n = x.numel()
    if with_bias:
        g = torch.Generator().manual_seed(7)
        bias = (torch.rand(n, generator=g) * 6.0 - 3.0).to(torch.float32)
        delta = x - bias                       # the kernel re-forms delta + bias in fp32
    else:
        bias, delta = None, x
    u = torch.ones(1, n, 1)
    dl = delta.view(1, n, 1).clone()
    A = -torch.ones(n, 1)
    Bm = torch.ones(1, 1, 1)
    Cm = torch.ones(1, 1, 1)
    dout = torch.ones(1, n, 1)

    ref = selective_scan_ref(u, dl, A, Bm, Cm, delta_bias=bias, delta_softplus=True)
    dl_ref = dl.clone().requires_grad_(True)
    selective_scan_ref(u, dl_ref, A, Bm, Cm, delta_bias=bias, delta_softplus=True).backward(dout)
    gref = dl_ref.grad

    dlg = dl.to(DEV).requires_grad_(True)
    out = s6scan.selective_scan_fn(u.to(DEV), dlg, A.to(DEV), Bm.to(DEV), Cm.to(DEV),
                                   delta_bias=None if bias is None else bias.to(DEV),
                                   delta_softplus=True)
    out.backward(dout.to(DEV))
    got, ggot = out.detach().cpu(), dlg.grad.cpu()

    for what, a, b in (("softplus", got, ref), ("softplus'", ggot, gref)):
        d = (a - b).abs()
        lim = 4 * _ulp32(b) + torch.finfo(torch.float32).tiny
        bad = d > lim
        i = int(torch.argmax((d - lim).flatten()))
        assert not bad.any(), (
            f"{what}: {int(bad.sum())}/{n} beyond 4 ulp; worst at x={x[i].item():.9g}: "
            f"got {a.flatten()[i].item():.9g} want {b.flatten()[i].item():.9g}")
    # the switch itself: above 20 softplus is the identity and its derivative exactly 1
    pre = x if bias is None else dl.flatten() + bias     # delta + bias as fp32 forms it
    above = pre > 20.0
    assert torch.equal(got.flatten()[above], pre[above])
    assert bool((ggot.flatten()[above] == 1.0).all())


def test_cfg2_kernel_no_farther_from_exact_than_fp32_restatement():
    """Config 2 (fp32, dstate 64, slow decay), full size on the GPU; on batch rows 0 and 15
    (full length) every output and final state satisfies
        |kernel - f64| <= |ref32 - f64| + 1e-6 + 1e-5 |f64|,
    f64 being the recurrence in float64 and ref32 the reference's fp32 evaluation order
    (selective_scan_interface.py:126-156, the C restatement).  The kernel is therefore within
    the north-star bar of wherever the reference's own fp32 result lands."""
    cfg = CONFIGS[2]
    i = make_inputs(cfg)
    g = {k: v.to(DEV) for k, v in i.items()}
    out, ls = s6scan.selective_scan_fn(g["x"].mT, g["delta"].mT, g["A"], g["B"].mT, g["C"].mT,
                                       D=g["D"], return_last_state=True)
    out, ls = out.cpu(), ls.cpu()
    del g
    report = []
    for b in (0, cfg.batch - 1):
        sl = slice(b, b + 1)
        args = (i["x"][sl].mT, i["delta"][sl].mT, i["A"], i["B"][sl].mT, i["C"][sl].mT)
        r32, rls32 = c_oracle.fwd(*args, D=i["D"])
        r64, rls64 = c_oracle.fwd64(*args, D=i["D"])
        for what, k, r, e in (("y", out[sl], r32, r64), ("last_state", ls[sl], rls32, rls64)):
            ek = (k.double() - e).abs()
            er = (r.double() - e).abs()
            lim = er + 1e-6 + 1e-5 * e.abs()
            bad = ek > lim
            report.append(f"row {b} {what}: max|k-f64| {ek.max().item():.3g}, "
                          f"max|ref32-f64| {er.max().item():.3g}, "
                          f"rms {ek.pow(2).mean().sqrt().item():.3g} vs "
                          f"{er.pow(2).mean().sqrt().item():.3g}")
            j = int(torch.argmax((ek - lim).flatten()))
            assert not bad.any(), (
                f"{what} row {b}: {int(bad.sum())}/{bad.numel()} elements farther from f64 than "
                f"the fp32 restatement + bar; worst: kernel {k.flatten()[j].item():.9g}, ref32 "
                f"{r.flatten()[j].item():.9g}, f64 {e.flatten()[j].item():.12g}")
    print("\n".join(report))


@pytest.mark.parametrize("path", ["lanes", "chunked"])
def test_bias_mode_fp32_no_farther_from_exact_than_reference_order(path, monkeypatch):
    """The bias-only delta mode in fp32 (large steps, strongly cancelling outputs, with the z
    gate) on both forward kernels.  The single-pass kernel rounds each C h product before
    its tree sum, as the reference's fp32 order does (selective_scan_interface.py:144: x * C,
    then the sum), so at cancelling outputs it lands about as far from the float64 value as
    the reference itself.  Every output and final state satisfies
        |kernel - f64| <= |ref32 - f64| + 1e-6 + 1e-5 |f64|."""
    from test_gpu_parity import call, gen

    monkeypatch.setenv("S6_FWD_PATH", path)
    inp = gen(2, 1203, 96, 16, torch.float32, seed=17, z=True, bias=True, softplus=False)
    args, kw = call(inp, "view", DEV)
    out, ls = s6scan.selective_scan_fn(*args, **kw)
    cargs, ckw = call(inp, "view", "cpu")
    okw = dict(D=ckw["D"], z=ckw["z"], delta_bias=ckw["delta_bias"], delta_softplus=False)
    r32, rls32 = c_oracle.fwd(*cargs, **okw)
    r64, rls64 = c_oracle.fwd64(*cargs, **okw)
    for what, k, r, e in (("y", out.cpu(), r32, r64), ("last_state", ls.cpu(), rls32, rls64)):
        ek = (k.double() - e).abs()
        er = (r.double() - e).abs()
        bad = ek > er + 1e-6 + 1e-5 * e.abs()
        assert not bad.any(), f"{path} {what}: {int(bad.sum())} elements; max |k-f64| {ek.max():.3g}"
