"""GPU parity of the causal conv1d kernels (s6scan.causal_conv1d) and the fused Mamba block
(s6scan.mamba_inner) against the CPU restatements in oracle/mamba_inner_ref.py (the
reference's nn.Conv1d path, mamba.py:159-161, and mamba_inner_ref,
selective_scan_interface.py:310-356), with gradients by autograd through the restatements."""
import pytest
import torch

import s6scan  # noqa: F401
from oracle.mamba_inner_ref import causal_conv1d_ref, mamba_inner_ref
from s6scan.causal_conv1d import causal_conv1d_bwd, causal_conv1d_fn, causal_conv1d_fwd
from s6scan.mamba_inner import MambaInnerFn, mamba_forward, mamba_inner_fn
from tolerances import assert_grad_close, assert_out_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_x(batch, dim, L, dtype, layout, g):
    """x [batch, dim, L] on the GPU: 'cl' channel-last, 'bdl' L-contiguous, 'half' the
    first half of a channel-last [batch, L, 2 dim] buffer (as in xz)."""
    if layout == "half":
        buf = torch.randn(batch, L, 2 * dim, generator=g).to(dtype)
        return buf.to(DEV).mT[:, :dim], buf.mT[:, :dim].float()
    x = torch.randn(batch, L, dim, generator=g).to(dtype)
    xg = x.to(DEV).mT if layout == "cl" else x.mT.contiguous().to(DEV)
    return xg, x.mT.float()


CONV_CASES = [  # (batch, dim, L, width, dtype, layout); channels per lane in the comments
    (2, 512, 300, 4, torch.bfloat16, "cl"),   # fwd 8, bwd 4
    (2, 1024, 70, 4, torch.float16, "half"),  # fwd 8, bwd 4
    (2, 256, 200, 3, torch.float32, "cl"),    # 4
    (1, 768, 129, 4, torch.bfloat16, "cl"),   # 4 (8 would idle a quarter of the lanes)
    (2, 64, 300, 4, torch.float32, "cl"),     # 1
    (2, 64, 300, 4, torch.bfloat16, "cl"),
    (2, 64, 300, 4, torch.float16, "cl"),
    (2, 64, 300, 4, torch.bfloat16, "bdl"),
    (2, 96, 257, 3, torch.bfloat16, "half"),  # 2
    (3, 20, 130, 2, torch.bfloat16, "cl"),    # dim % 8 != 0: one channel per lane
    (3, 20, 130, 2, torch.float32, "cl"),     # dim % 4 == 0: fp32 vector path
    (1, 72, 1, 4, torch.float32, "cl"),       # seqlen 1
    (2, 16, 3, 4, torch.bfloat16, "cl"),      # seqlen < width
    (1, 1040, 2100, 4, torch.bfloat16, "cl"),  # 2; several channel and sequence blocks
]


@pytest.mark.parametrize("silu", [True, False])
@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_forward_matches_reference(case, silu):
    batch, dim, L, W, dtype, layout = case
    g = torch.Generator().manual_seed(dim * 7 + L)
    x, xr = make_x(batch, dim, L, dtype, layout, g)
    w = torch.randn(dim, W, generator=g) * 0.5
    b = torch.randn(dim, generator=g)
    out = causal_conv1d_fwd(x, w.to(DEV), b.to(DEV), None, None, None, silu)
    assert out.dtype == dtype and out.shape == x.shape
    if layout != "bdl":
        assert out.stride(1) == 1, "output must follow the channel-last input layout"
    ref = causal_conv1d_ref(xr.double(), w.double(), b.double(), "silu" if silu else None)
    assert_out_close(out, ref, dtype, "conv out")


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_backward_matches_autograd(case):
    batch, dim, L, W, dtype, layout = case
    g = torch.Generator().manual_seed(dim * 11 + L)
    x, xr = make_x(batch, dim, L, dtype, layout, g)
    w = torch.randn(dim, W, generator=g) * 0.5
    b = torch.randn(dim, generator=g)
    dout = torch.randn(batch, L, dim, generator=g).to(dtype)
    dx, dw, db, dinit = causal_conv1d_bwd(x, w.to(DEV), b.to(DEV), dout.to(DEV).mT, None, None,
                                          None, None, False, True)
    assert dinit is None and dx.shape == x.shape and dx.dtype == dtype
    xl = xr.double().requires_grad_(True)
    wl = w.double().requires_grad_(True)
    bl = b.double().requires_grad_(True)
    y = causal_conv1d_ref(xl, wl, bl, "silu")
    gx, gw, gb = torch.autograd.grad((y * dout.mT.double()).sum(), (xl, wl, bl))
    assert_grad_close(dx, gx, dtype, "dx")
    assert_grad_close(dw, gw, dtype, "dweight")
    assert_grad_close(db, gb, dtype, "dbias")


def test_conv_backward_long_sequence_reduces_partials_in_order():
    """seqlen long enough that each block walks several tiles and many partial rows are
    reduced; run twice to check the reduction is deterministic."""
    batch, dim, L, W = 1, 64, 256 * 2100, 4
    g = torch.Generator().manual_seed(5)
    x = torch.randn(batch, L, dim, generator=g)
    w = torch.randn(dim, W, generator=g) * 0.5
    b = torch.randn(dim, generator=g)
    dout = torch.randn(batch, L, dim, generator=g)
    args = (x.to(DEV).mT, w.to(DEV), b.to(DEV), dout.to(DEV).mT)
    r1 = causal_conv1d_bwd(*args, silu_activation=True)
    r2 = causal_conv1d_bwd(*args, silu_activation=True)
    for a1, a2 in zip(r1[:3], r2[:3]):
        assert torch.equal(a1, a2)
    xl = x.mT.double().requires_grad_(True)
    wl = w.double().requires_grad_(True)
    bl = b.double().requires_grad_(True)
    y = causal_conv1d_ref(xl, wl, bl, "silu")
    gx, gw, gb = torch.autograd.grad((y * dout.mT.double()).sum(), (xl, wl, bl))
    assert_grad_close(r1[0], gx, torch.float32, "dx")
    assert_grad_close(r1[1], gw, torch.float32, "dweight")
    assert_grad_close(r1[2], gb, torch.float32, "dbias")


def test_conv_module_arities_as_each_reference_file_calls_them():
    """The two copies of the reference's interface file call the conv module with different
    argument lists: the ops copy with the newer ones (selective_scan_interface.py:187-189,
    299-301: fwd with 7 arguments, bwd with 10 returning 4 values) and the copy zoology's
    Mamba imports (mamba_ssm/selective_scan_interface.py:181, 288-290, 321: fwd with 5, bwd with
    7 returning 3 values, causal_conv1d_fn with the activation 4th).  s6scan.causal_conv1d
    serves the first, s6scan.causal_conv1d_legacy the second; both must equal the reference's
    nn.Conv1d path and its autograd."""
    from s6scan import causal_conv1d as conv_new
    from s6scan import causal_conv1d_legacy as conv_old

    g = torch.Generator().manual_seed(21)
    batch, dim, L, W = 2, 160, 257, 4
    xz = torch.randn(batch, L, 2 * dim, generator=g).to(torch.bfloat16)
    x = xz.to(DEV).mT[:, :dim]                       # x half of a channel-last xz, as in the block
    xr = xz.mT[:, :dim].double()
    w = torch.randn(dim, W, generator=g) * 0.5
    b = torch.randn(dim, generator=g)
    dout = torch.randn(batch, L, dim, generator=g).to(torch.bfloat16)
    wg, bg, doutg = w.to(DEV), b.to(DEV), dout.to(DEV).mT

    ref = causal_conv1d_ref(xr, w.double(), b.double(), "silu")
    xl = xr.clone().requires_grad_(True)
    wl = w.double().requires_grad_(True)
    bl = b.double().requires_grad_(True)
    gx, gw, gb = torch.autograd.grad(
        (causal_conv1d_ref(xl, wl, bl, "silu") * dout.mT.double()).sum(), (xl, wl, bl))

    # ops copy: conv1d_out = causal_conv1d_fwd(x, w, b, None, None, None, True)
    out_new = conv_new.causal_conv1d_fwd(x, wg, bg, None, None, None, True)
    # Mamba's copy: conv1d_out = causal_conv1d_fwd(x, w, b, None, True)
    out_old = conv_old.causal_conv1d_fwd(x, wg, bg, None, True)
    assert torch.equal(out_new, out_old)
    assert_out_close(out_old, ref, torch.bfloat16, "conv out (5-argument fwd)")

    # ops copy: dx, dw, db, *_ = causal_conv1d_bwd(x, w, b, dout, None, None, None, dx, False, True)
    dx_new = torch.empty_like(x)
    res_new = conv_new.causal_conv1d_bwd(x, wg, bg, doutg, None, None, None, dx_new, False, True)
    assert len(res_new) == 4 and res_new[0] is dx_new
    # Mamba's copy: dx, dw, db = causal_conv1d_bwd(x, w, b, dout, None, dx, True)
    dx_old = torch.empty_like(x)
    res_old = conv_old.causal_conv1d_bwd(x, wg, bg, doutg, None, dx_old, True)
    assert len(res_old) == 3 and res_old[0] is dx_old
    for a_new, a_old in zip(res_new[:3], res_old):
        assert torch.equal(a_new, a_old)
    assert_grad_close(res_old[0], gx, torch.bfloat16, "dx (7-argument bwd)")
    assert_grad_close(res_old[1], gw, torch.bfloat16, "dweight (7-argument bwd)")
    assert_grad_close(res_old[2], gb, torch.bfloat16, "dbias (7-argument bwd)")

    # causal_conv1d_fn: activation 4th (Mamba's copy, :321) and 5th (mamba.py:163-169)
    y_old = conv_old.causal_conv1d_fn(x, wg, bg, "silu")
    y_new = conv_new.causal_conv1d_fn(x, wg, bg, None, "silu")
    assert torch.equal(y_old, y_new)
    assert_out_close(y_old, ref, torch.bfloat16, "causal_conv1d_fn")


def test_conv_fn_autograd_without_bias():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 100, 32, generator=g)
    w = torch.randn(32, 3, generator=g)
    xg = x.to(DEV).mT.requires_grad_(True)
    wg = w.to(DEV).requires_grad_(True)
    y = causal_conv1d_fn(xg, wg, None, None, "swish")
    dy = torch.randn(y.shape, generator=g)
    y.backward(dy.to(DEV))
    xl = x.mT.double().requires_grad_(True)
    wl = w.double().requires_grad_(True)
    yr = causal_conv1d_ref(xl, wl, None, "silu")
    yr.backward(dy.double())
    assert_out_close(y, yr, torch.float32)
    assert_grad_close(xg.grad, xl.grad, torch.float32, "dx")
    assert_grad_close(wg.grad, wl.grad, torch.float32, "dweight")


def test_conv_rejects_what_the_reference_path_never_passes():
    x = torch.zeros(1, 8, 16, device=DEV)
    w = torch.zeros(8, 4, device=DEV)
    with pytest.raises(NotImplementedError):
        causal_conv1d_fwd(x, w, None, torch.zeros(1, 16, dtype=torch.int32, device=DEV))
    with pytest.raises(NotImplementedError):
        causal_conv1d_fwd(x, torch.zeros(8, 5, device=DEV), None)
    with pytest.raises(NotImplementedError):
        causal_conv1d_fn(x, w, None, None, "relu")


# ---- fused block ------------------------------------------------------------------------

def block_params(seed, batch=2, L=300, d_model=64, d_inner=128, d_state=16, dt_rank=4,
                 width=4, proj_bias=True):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=1.0: torch.randn(*s, generator=g) * sc
    A_log = torch.log(torch.arange(1, d_state + 1, dtype=torch.float32))[None].repeat(d_inner, 1)
    p = dict(
        xz=r(batch, L, 2 * d_inner).mT,  # values; layout chosen per test
        conv1d_weight=r(d_inner, 1, width, sc=0.5), conv1d_bias=r(d_inner, sc=0.5),
        x_proj_weight=r(dt_rank + 2 * d_state, d_inner, sc=d_inner ** -0.5),
        delta_proj_weight=r(d_inner, dt_rank, sc=dt_rank ** -0.5),
        out_proj_weight=r(d_model, d_inner, sc=d_inner ** -0.5), out_proj_bias=r(d_model, sc=0.1),
        A=-torch.exp(A_log + 0.1 * r(d_inner, d_state)), D=r(d_inner),
        delta_bias=torch.log(torch.expm1(torch.rand(d_inner, generator=g) * 0.09 + 0.01)),
        B_proj_bias=r(d_state, sc=0.1) if proj_bias else None,
        C_proj_bias=r(d_state, sc=0.1) if proj_bias else None)
    return p


ORDER = ["xz", "conv1d_weight", "conv1d_bias", "x_proj_weight", "delta_proj_weight",
         "out_proj_weight", "out_proj_bias", "A", "B", "C", "D", "delta_bias", "B_proj_bias",
         "C_proj_bias"]


def run_block(p, dev, fn, layout="cl", ckpt=None):
    leaves = {k: v.detach().clone().to(dev).requires_grad_(True)
              for k, v in p.items() if v is not None}
    if dev == DEV and layout == "cl":
        leaves["xz"] = p["xz"].mT.contiguous().to(dev).mT.detach().requires_grad_(True)
    elif dev == DEV:
        leaves["xz"] = p["xz"].contiguous().to(dev).requires_grad_(True)
    args = [leaves.get(k) for k in ORDER] + [True]
    if ckpt is not None:
        out = MambaInnerFn.apply(*args, ckpt)
    else:
        out = fn(*args)
    return out, leaves


@pytest.mark.parametrize("ckpt", [None, 0])
@pytest.mark.parametrize("layout", ["cl", "bdl"])
@pytest.mark.parametrize("proj_bias", [True, False])
def test_mamba_inner_fn_matches_reference(layout, proj_bias, ckpt):
    p = block_params(3, proj_bias=proj_bias)
    out, lg = run_block(p, DEV, mamba_inner_fn, layout, ckpt)
    ref, lc = run_block(p, "cpu", mamba_inner_ref)
    assert out.shape == ref.shape == (2, 300, 64)
    assert_out_close(out, ref, torch.float32, "out", dstate=16)
    dy = torch.randn(out.shape, generator=torch.Generator().manual_seed(4))
    out.backward(dy.to(DEV))
    ref.backward(dy)
    for k in lc:
        assert lg[k].grad is not None, k
        assert_grad_close(lg[k].grad, lc[k].grad, torch.float32, "d" + k)


def test_mamba_inner_fn_bf16_autocast():
    """Training configuration: bf16 activations, fp32 parameters, autocast GEMMs.  The GPU
    result is compared norm-wise with the fp32 reference."""
    p = block_params(6, L=256)
    lg = {k: v.detach().clone().to(DEV).requires_grad_(True) for k, v in p.items()}
    lg["xz"] = p["xz"].mT.contiguous().to(DEV, torch.bfloat16).mT.detach().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = mamba_inner_fn(*[lg.get(k) for k in ORDER], True)
    assert out.dtype == torch.bfloat16
    ref, lc = run_block(dict(p, xz=p["xz"].to(torch.bfloat16).float()), "cpu", mamba_inner_ref)
    dy = torch.randn(out.shape, generator=torch.Generator().manual_seed(7))
    out.float().backward(dy.to(DEV))
    ref.backward(dy)

    def rel(a, b):
        a, b = a.detach().float().cpu(), b.detach().float()
        return ((a - b).norm() / b.norm()).item()

    assert rel(out, ref) < 2e-2, rel(out, ref)
    for k in lc:
        assert rel(lg[k].grad, lc[k].grad) < 5e-2, (k, rel(lg[k].grad, lc[k].grad))


class _ZooMamba(torch.nn.Module):
    """The parameters of the reference's zoology Mamba (mamba.py:22-100) by their names."""

    def __init__(self, d_model, d_state=16, d_conv=4, expand=2, seed=0):
        super().__init__()
        torch.manual_seed(seed)
        d_inner = expand * d_model
        self.dt_rank = -(-d_model // 16)
        self.in_proj = torch.nn.Linear(d_model, 2 * d_inner, bias=False)
        self.conv1d = torch.nn.Conv1d(d_inner, d_inner, d_conv, groups=d_inner,
                                      padding=d_conv - 1)
        self.x_proj = torch.nn.Linear(d_inner, self.dt_rank + 2 * d_state, bias=False)
        self.dt_proj = torch.nn.Linear(self.dt_rank, d_inner, bias=True)
        self.out_proj = torch.nn.Linear(d_inner, d_model, bias=False)
        self.A_log = torch.nn.Parameter(
            torch.log(torch.arange(1, d_state + 1, dtype=torch.float32)).repeat(d_inner, 1))
        self.D = torch.nn.Parameter(torch.ones(d_inner))


def test_mamba_forward_matches_reference_fast_path():
    m = _ZooMamba(64, seed=11)
    h = torch.randn(2, 200, 64, generator=torch.Generator().manual_seed(12))
    mg = _ZooMamba(64, seed=11).to(DEV)
    out = mamba_forward(mg, h.to(DEV))
    # the reference's fast path (mamba.py:125-153) with the restated mamba_inner_ref
    xz = (m.in_proj.weight @ h.reshape(-1, 64).t()).reshape(256, 2, 200).permute(1, 0, 2)
    ref = mamba_inner_ref(xz, m.conv1d.weight, m.conv1d.bias, m.x_proj.weight, m.dt_proj.weight,
                          m.out_proj.weight, m.out_proj.bias, -torch.exp(m.A_log.float()), None,
                          None, m.D.float(), delta_bias=m.dt_proj.bias.float(),
                          delta_softplus=True)
    assert_out_close(out, ref, torch.float32, "mamba out", dstate=16)
    out.sum().backward()
    ref.sum().backward()
    for (n, pg), (_, pc) in zip(mg.named_parameters(), m.named_parameters()):
        assert_grad_close(pg.grad, pc.grad, torch.float32, n)


@pytest.mark.parametrize("shape", [(65536, 56, 768), (65536, 768, 24), (65536, 384, 768), (6144, 40, 96)])
def test_split_weight_gradient_matches_float64(shape):
    """The block's weight gradients a.t() @ b over T = batch * seqlen tokens run split over T
    (fp32 partials summed in a fixed order, one rounding); compare with float64, in fp32 and
    under bf16 autocast (where the single product's own rounding to bf16 is the bound)."""
    from s6scan.mamba_inner import _wgrad
    T, M, N = shape
    g = torch.Generator().manual_seed(M + N)
    a, b = torch.randn(T, M, generator=g), torch.randn(T, N, generator=g)
    ref = a.double().t() @ b.double()
    scale = ref.abs().max().item()
    got = _wgrad(a.to(DEV), b.to(DEV))
    assert got.dtype == torch.float32 and got.shape == (M, N)
    assert (got.double().cpu() - ref).abs().max().item() <= 1e-5 * scale
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ab, bb = a.to(DEV, torch.bfloat16), b.to(DEV, torch.bfloat16)
        got16 = _wgrad(ab, bb)
        one = ab.t() @ bb  # the single product the split replaces
    assert got16.dtype == torch.bfloat16
    ref16 = ab.double().cpu().t() @ bb.double().cpu()
    err = (got16.double().cpu() - ref16).abs()
    assert err.max().item() <= 2 ** -8 * ref16.abs().max().item()  # one bf16 rounding
    assert err.norm().item() <= 1.05 * (one.double().cpu() - ref16).norm().item() + 1e-6


def test_mamba_inner_fn_long_sequence_split_weight_grads():
    """T = 2 * 2048 tokens: the weight gradients take the split path (S = 2)."""
    p = block_params(21, batch=2, L=2048, d_model=32, d_inner=64, dt_rank=2, proj_bias=False)
    out, lg = run_block(p, DEV, mamba_inner_fn, "cl")
    ref, lc = run_block(p, "cpu", mamba_inner_ref)
    assert_out_close(out, ref, torch.float32, "out", dstate=16)
    dy = torch.randn(out.shape, generator=torch.Generator().manual_seed(22))
    out.backward(dy.to(DEV))
    ref.backward(dy)
    for k in ("x_proj_weight", "delta_proj_weight", "out_proj_weight", "xz", "A", "D"):
        assert_grad_close(lg[k].grad, lc[k].grad, torch.float32, "d" + k)


def test_in_proj_split_weight_gradient_matches_autograd():
    """InProjFn (mamba_forward's in_proj) against autograd's F.linear, fp32 and bf16 autocast,
    at T = 4096 tokens so the weight gradient takes the split path."""
    from s6scan.mamba_inner import InProjFn
    g = torch.Generator().manual_seed(31)
    h = torch.randn(4096, 48, generator=g).to(DEV)
    w = (torch.randn(96, 48, generator=g) * 0.1).to(DEV)
    bias = (torch.randn(96, generator=g) * 0.1).to(DEV)
    dy = torch.randn(4096, 96, generator=g).to(DEV)
    for ac in (False, True):
        leaves = [t.clone().requires_grad_(True) for t in (h, w, bias)]
        refs = [t.clone().requires_grad_(True) for t in (h, w, bias)]
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=ac):
            out = InProjFn.apply(*leaves)
            ref = torch.nn.functional.linear(*refs)
        assert out.dtype == ref.dtype
        out.backward(dy.to(out.dtype))
        ref.backward(dy.to(ref.dtype))
        for a, b, name in zip(leaves, refs, ("dh", "dw", "db")):
            assert a.grad.dtype == b.grad.dtype, name
            tol = 1e-5 if not ac else 1e-2
            err = ((a.grad - b.grad).float().norm() / b.grad.float().norm()).item()
            assert err <= tol, (name, ac, err)
