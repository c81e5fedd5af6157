"""GPU parity of the Mamba-2 SSD forward (s6scan.ssd_combined) against the CPU restatement of
the reference's chunked pipeline (oracle/ssd_ref.py, pinned by its float64 brute force),
computed in float64 on the same (16-bit-rounded) inputs."""
import numpy as np
import pytest
import torch

import s6scan  # noqa: F401
from oracle.ssd_ref import ssd_chunked_ref
from s6scan.ssd_combined import mamba_chunk_scan_combined, ssd_forward
from tolerances import assert_close, rms

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(batch, L, H, P, G, N, dtype, seed, opts=()):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    t = dict(x=r(batch, L, H, P).to(dtype), dt=(0.5 * r(batch, L, H) - 1.0).to(dtype),
             A=-torch.exp(torch.rand(H, generator=g) * 2.77),  # A in [-16, -1] as Mamba-2's init
             B=r(batch, L, G, N).to(dtype), C=r(batch, L, G, N).to(dtype))
    kw = dict(dt_softplus=True)
    if "D" in opts:
        t["D"] = r(H)
    if "D_hdim" in opts:
        t["D"] = r(H, P)
    if "z" in opts:
        t["z"] = r(batch, L, H, P).to(dtype)
    if "bias" in opts:
        t["dt_bias"] = 0.5 * r(H)
    if "init" in opts:
        t["initial_states"] = r(batch, H, P, N)
    if "seq" in opts:
        seq = torch.zeros(batch, L, dtype=torch.int32)
        for b in range(batch):
            cuts = sorted(torch.randint(1, L, (3,), generator=g).tolist())
            for i, cpos in enumerate(cuts):
                seq[b, cpos:] = i + 1
        t["seq_idx"] = seq
    if "limit" in opts:
        kw["dt_limit"] = (0.05, 0.5)
    return t, kw


def check(out, ref, dtype, what):
    if dtype == torch.float32:
        assert_close(out, ref, 1e-4, 1e-4 * rms(ref), what)
    else:  # the scaled B, the decayed CB and the passed states are rounded to the 16-bit type
        # (as in the reference); compare norm-wise and elementwise against the float64 value
        # (fp16 keeps 3 more mantissa bits than bf16, so its bounds are 8x tighter)
        k = 1.0 if dtype == torch.bfloat16 else 0.125
        d = (out.float().cpu() - ref.float())
        rel = (d.norm() / ref.float().norm()).item()
        assert rel < 1.5e-2 * k, f"{what}: norm-wise relative error {rel:.3g}"
        assert_close(out, ref, 5e-2 * k, 5e-2 * k * rms(ref), what)


CASES = [  # batch, L, H, P, G, N, chunk, opts
    (2, 300, 4, 64, 2, 64, 64, ("D", "z", "bias")),
    (1, 512, 2, 32, 1, 128, 128, ("init", "seq", "D")),
    (2, 256, 3, 128, 3, 32, 256, ("D_hdim", "limit", "bias")),
    (1, 1000, 2, 64, 1, 256, 256, ("z", "init")),
    (2, 190, 8, 64, 1, 128, 64, ("seq", "init", "z", "D", "bias")),
    (1, 64, 1, 32, 1, 32, 64, ()),
    # workgroup counts that are not multiples of the 8 XCDs (54 chunk-scan blocks, 27
    # dCB tiles, 18 row blocks): the uneven branch of the XCD work mapping
    (3, 330, 3, 64, 1, 64, 128, ("D", "bias", "z")),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", CASES)
def test_ssd_forward_matches_reference(case, dtype):
    batch, L, H, P, G, N, Q, opts = case
    t, kw = make(batch, L, H, P, G, N, dtype, seed=L + N, opts=opts)
    gpu = {k: v.to(DEV) for k, v in t.items()}
    out, out_x, final, _ = ssd_forward(**gpu, chunk_size=Q, want_final_states=True,
                                    want_out_x=True, **kw)
    ref, ref_x, ref_final = ssd_chunked_ref(**t, chunk_size=Q, compute_dtype=torch.float64, **kw)
    assert out.shape == (batch, L, H, P) and out.dtype == dtype
    check(out, ref, dtype, "out")
    if "z" in opts:
        check(out_x, ref_x, dtype, "out_x")
    check(final, ref_final, torch.float32 if dtype == torch.float32 else dtype, "final_states")


def test_ssd_mamba2_defaults_bf16():
    """Mamba-2's default layer: headdim 64, dstate 128, chunk 256, one group, D per head,
    dt bias + softplus, no z (the RMSNorm variant); x, B, C are views of one xBC buffer."""
    batch, L, H, P, N = 2, 1024, 8, 64, 128
    g = torch.Generator().manual_seed(17)
    xBC = torch.randn(batch, L, H * P + 2 * N, generator=g).to(torch.bfloat16)
    x = xBC[..., :H * P].reshape(batch, L, H, P)
    B = xBC[..., H * P:H * P + N].reshape(batch, L, 1, N)
    C = xBC[..., H * P + N:].reshape(batch, L, 1, N)
    dt = (0.5 * torch.randn(batch, L, H, generator=g) - 2.0).to(torch.bfloat16)
    A = -torch.exp(torch.rand(H, generator=g) * 2.77)
    D, bias = torch.randn(H, generator=g), 0.3 * torch.randn(H, generator=g)
    dv = lambda v: v.to(DEV)
    xg = dv(xBC)
    out = mamba_chunk_scan_combined(
        xg[..., :H * P].reshape(batch, L, H, P), dv(dt), dv(A),
        xg[..., H * P:H * P + N].reshape(batch, L, 1, N), xg[..., H * P + N:].reshape(batch, L, 1, N),
        256, D=dv(D), dt_bias=dv(bias), dt_softplus=True)
    ref, _, _ = ssd_chunked_ref(x, dt, A, B, C, 256, D=D, dt_bias=bias, dt_softplus=True,
                                compute_dtype=torch.float64)
    check(out, ref, torch.bfloat16, "out")


@pytest.mark.parametrize("shape,what", [((160, 32, 64), "headdim"), ((64, 300, 64), "dstate"),
                                        ((64, 32, 32), "chunk_size"), ((64, 32, 100), "chunk_size")])
def test_ssd_rejects_unsupported_shapes(shape, what):
    P, N, Q = shape
    t, kw = make(1, 64, 1, P, 1, N, torch.float32, seed=1)
    with pytest.raises(RuntimeError, match=what):
        ssd_forward(**{k: v.to(DEV) for k, v in t.items()}, chunk_size=Q, **kw)


# Shapes off the kernels' tiles (headdim 32 / 64 / 128, dstate 32 / 64 / 128 / 256), which run
# on zero-padded copies: zoology's Mamba-2 sweep (models_repo.py:131-137: d_state 8 / 16 / 24,
# mamba2.py:35-53: headdim 64, chunk_size 256; d_model 64 / 128 / 256 give 2 / 4 / 8 heads),
# chunk 64, other headdims, and chunk 192.
PAD_CASES = [  # batch, L, H, P, G, N, chunk, opts
    (2, 256, 4, 64, 1, 16, 256, ("D", "bias", "final")),
    (2, 300, 2, 64, 1, 24, 64, ("z", "D", "bias", "init", "final")),
    (1, 700, 8, 64, 1, 8, 256, ("D_hdim", "seq", "bias")),
    (2, 333, 4, 64, 2, 24, 256, ("z", "bias", "limit")),
    (2, 200, 4, 48, 2, 16, 64, ("z", "D_hdim", "init", "final")),
    (1, 400, 3, 80, 1, 40, 192, ("D", "bias", "seq", "final")),
    (2, 130, 2, 24, 1, 100, 128, ("z", "init", "final", "limit")),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", PAD_CASES, ids=lambda c: "-".join(map(str, c[:7])))
def test_ssd_padded_shapes_forward_and_backward(case, dtype):
    batch, L, H, P, G, N, Q, opts = case
    t, kw = make(batch, L, H, P, G, N, dtype, seed=L + 7 * N + P, opts=opts)
    final = "final" in opts
    g = torch.Generator().manual_seed(L + 2)
    dy = torch.randn(batch, L, H, P, generator=g)
    dfin = torch.randn(batch, H, P, N, generator=g)
    names = [k for k, v in t.items() if v.is_floating_point()]
    gpu = {k: (v.to(DEV).requires_grad_(True) if k in names else v.to(DEV)) for k, v in t.items()}
    res = mamba_chunk_scan_combined(**gpu, chunk_size=Q, return_final_states=final, **kw)
    out, fin = res if final else (res, None)
    cpu = {k: (v.double().requires_grad_(True) if k in names else v) for k, v in t.items()}
    ref, _, ref_fin = ssd_chunked_ref(**cpu, chunk_size=Q, compute_dtype=torch.float64, **kw)
    assert out.shape == (batch, L, H, P) and out.dtype == dtype
    check(out, ref.detach(), dtype, "out")
    if final:
        assert fin.shape == (batch, H, P, N)
        check(fin, ref_fin.detach(), torch.float32 if dtype == torch.float32 else dtype, "final_states")
    loss = (out.float() * dy.to(DEV)).sum() + ((fin * dfin.to(DEV)).sum() if final else 0.0)
    loss.backward()
    rloss = (ref * dy.double()).sum() + ((ref_fin * dfin.double()).sum() if final else 0.0)
    rloss.backward()
    if dtype == torch.float32:
        # dA and ddt_bias sum over every step of the batch with heavy cancellation, so their
        # fp32 error depends on the order of the sum: the bound adds twice the worst error of
        # the reference's own fp32 evaluation (the same restatement in float32 autograd)
        c32 = {k: (v.detach().clone().requires_grad_(True) if k in names else v) for k, v in t.items()}
        r32, _, r32_fin = ssd_chunked_ref(**c32, chunk_size=Q, compute_dtype=torch.float32, **kw)
        ((r32 * dy).sum() + ((r32_fin * dfin).sum() if final else 0.0)).backward()
    for k in names:
        assert gpu[k].grad.shape == t[k].shape and gpu[k].grad.dtype == t[k].dtype, k
        if dtype == torch.float32:
            e32 = (c32[k].grad.double() - cpu[k].grad).abs().max().item()
            ref_g = cpu[k].grad
            assert_close(gpu[k].grad, ref_g, 1e-4, 1e-4 * rms(ref_g) + 2 * e32, "d" + k)
        else:
            check_grad(gpu[k].grad, cpu[k].grad, dtype, "d" + k)


def test_ssd_padded_shapes_strided_views():
    """Padded shapes read any strides: x, B, C as views of one [batch, L, H P + 2 G N] buffer
    whose rows are not 16-byte multiples (headdim 40, dstate 12, bf16), and out_x / z through
    the z gate; the result equals the one from contiguous copies bit for bit."""
    batch, L, H, P, G, N = 2, 260, 2, 40, 1, 12
    g = torch.Generator().manual_seed(9)
    buf = torch.randn(batch, L, H * P + 2 * G * N + 3, generator=g).to(torch.bfloat16).to(DEV)
    x = buf[..., 3:3 + H * P].unflatten(-1, (H, P))
    B = buf[..., 3 + H * P:3 + H * P + G * N].unflatten(-1, (G, N))
    C = buf[..., 3 + H * P + G * N:].unflatten(-1, (G, N))
    dt = (0.5 * torch.randn(batch, L, H, generator=g) - 1.0).to(torch.bfloat16).to(DEV)
    A = (-torch.exp(torch.rand(H, generator=g) * 2.77)).to(DEV)
    z = torch.randn(batch, L, H, P, generator=g).to(torch.bfloat16).to(DEV)
    kw = dict(D=torch.randn(H, generator=g).to(DEV), dt_softplus=True)
    a = mamba_chunk_scan_combined(x, dt, A, B, C, 64, z=z, **kw)
    b = mamba_chunk_scan_combined(x.contiguous(), dt, A, B.contiguous(), C.contiguous(), 64, z=z, **kw)
    assert torch.equal(a, b)
    ref, _, _ = ssd_chunked_ref(x.cpu(), dt.cpu(), A.cpu(), B.cpu(), C.cpu(), 64, z=z.cpu(),
                                D=kw["D"].cpu(), dt_softplus=True, compute_dtype=torch.float64)
    check(a, ref, torch.bfloat16, "out")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ssd_varlen_states_padded_shapes(dtype):
    from oracle.ssd_ref import ssd_varlen_states_ref
    cu = [0, 50, 64, 200, 201, 513, 700]
    t, kw = make(1, 700, 2, 48, 1, 24, dtype, seed=78, opts=("bias", "D", "init"))
    gpu = {k: v.to(DEV) for k, v in t.items()}
    out, vst = mamba_chunk_scan_combined(
        **gpu, chunk_size=64, cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=DEV),
        return_varlen_states=True, **kw)
    assert vst.shape == (len(cu) - 1, 2, 48, 24) and vst.dtype == dtype
    ref = ssd_varlen_states_ref(t["x"].double(), t["dt"].double(), t["A"].double(),
                                t["B"].double(), 64, torch.tensor(cu),
                                dt_bias=t["dt_bias"].double(),
                                initial_states=t["initial_states"].double(),
                                compute_dtype=torch.float64, **kw)
    check(vst, ref, dtype, "varlen_states")


GRAD_CASES = [  # batch, L, H, P, G, N, chunk, opts
    (2, 300, 4, 64, 2, 64, 64, ("D", "z", "bias")),
    (1, 512, 2, 32, 1, 128, 128, ("init", "seq", "D_hdim", "final")),
    (2, 256, 3, 128, 3, 32, 256, ("limit", "bias")),
    (1, 200, 2, 64, 1, 256, 64, ("z", "init", "bias", "final")),
    (2, 130, 4, 32, 2, 32, 64, ("seq", "z", "D")),
    (3, 330, 3, 64, 1, 64, 128, ("D", "bias", "init", "final")),
]


def check_grad(a, b, dtype, what):
    if dtype == torch.float32:
        assert_close(a, b, 1e-4, 1e-4 * rms(b), what)
    else:
        d = a.detach().float().cpu() - b.detach().float()
        rel = (d.norm() / b.detach().float().norm()).item()
        bound = 3e-2 if dtype == torch.bfloat16 else 3e-2 / 8
        assert rel < bound, f"{what}: norm-wise relative error {rel:.3g}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", GRAD_CASES)
def test_ssd_backward_matches_autograd(case, dtype):
    batch, L, H, P, G, N, Q, opts = case
    t, kw = make(batch, L, H, P, G, N, dtype, seed=L + 3 * N, opts=opts)
    final = "final" in opts
    g = torch.Generator().manual_seed(L)
    dy = torch.randn(batch, L, H, P, generator=g)
    dfin = torch.randn(batch, H, P, N, generator=g)
    names = [k for k, v in t.items() if v.is_floating_point()]
    gpu = {k: (v.to(DEV).requires_grad_(True) if k in names else v.to(DEV)) for k, v in t.items()}
    res = mamba_chunk_scan_combined(**gpu, chunk_size=Q, return_final_states=final, **kw)
    out, fin = res if final else (res, None)
    loss = (out.float() * dy.to(DEV)).sum() + ((fin * dfin.to(DEV)).sum() if final else 0.0)
    loss.backward()
    cpu = {k: (v.double().requires_grad_(True) if k in names else v) for k, v in t.items()}
    ref, _, ref_fin = ssd_chunked_ref(**cpu, chunk_size=Q, compute_dtype=torch.float64, **kw)
    rloss = (ref * dy.double()).sum() + ((ref_fin * dfin.double()).sum() if final else 0.0)
    rloss.backward()
    for k in names:
        assert gpu[k].grad is not None, k
        assert gpu[k].grad.shape == t[k].shape and gpu[k].grad.dtype == t[k].dtype, k
        check_grad(gpu[k].grad, cpu[k].grad, dtype, "d" + k)


def test_ssd_backward_is_deterministic():
    t, kw = make(2, 300, 4, 64, 2, 64, torch.bfloat16, seed=5, opts=("D", "z", "bias", "init"))
    dy = torch.randn(2, 300, 4, 64, generator=torch.Generator().manual_seed(6)).to(DEV)
    grads = []
    for _ in range(2):
        gpu = {k: v.to(DEV).requires_grad_(True) for k, v in t.items()}
        out = mamba_chunk_scan_combined(**gpu, chunk_size=64, **kw)
        (out.float() * dy).sum().backward()
        grads.append([gpu[k].grad.clone() for k in sorted(gpu)])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


VCU = [0, 50, 64, 200, 201, 513, 700]  # chunk 64: ends on a boundary, carries, length 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_seq", [True, False])
def test_ssd_varlen_states_match_reference(dtype, with_seq):
    from oracle.ssd_ref import ssd_varlen_states_ref
    t, kw = make(1, 700, 3, 32, 1, 32, dtype, seed=77, opts=("bias", "D", "init"))
    seq = torch.zeros(1, 700, dtype=torch.int32)
    for i, (s0, s1) in enumerate(zip(VCU[:-1], VCU[1:])):
        seq[0, s0:s1] = i
    if with_seq:
        t["seq_idx"] = seq
    gpu = {k: v.to(DEV) for k, v in t.items()}
    out, final, vst = mamba_chunk_scan_combined(
        **gpu, chunk_size=64, cu_seqlens=torch.tensor(VCU, dtype=torch.int32, device=DEV),
        return_final_states=True, return_varlen_states=True, **kw)
    assert vst.shape == (len(VCU) - 1, 3, 32, 32) and vst.dtype == dtype
    ref = ssd_varlen_states_ref(t["x"].double(), t["dt"].double(), t["A"].double(),
                                t["B"].double(), 64, torch.tensor(VCU),
                                dt_bias=t["dt_bias"].double(),
                                initial_states=t["initial_states"].double(),
                                seq_idx=t.get("seq_idx"), compute_dtype=torch.float64, **kw)
    check(vst, ref, dtype, "varlen_states")
    # the last sequence ends at the end of the input: its state is the final state
    if with_seq:
        check(final[0].float(), ref[-1], torch.float32 if dtype == torch.float32 else dtype, "final")


def test_ssd_varlen_states_argument_rules():
    """The reference's asserts (ssd_combined.py:329, 540, 557)."""
    t, kw = make(2, 128, 2, 32, 1, 32, torch.float32, seed=5)
    gpu = {k: v.to(DEV) for k, v in t.items()}
    cu = torch.tensor([0, 100, 128], dtype=torch.int32, device=DEV)
    with pytest.raises(AssertionError, match="batch dimension is 1"):
        mamba_chunk_scan_combined(**gpu, chunk_size=64, cu_seqlens=cu, return_varlen_states=True, **kw)
    one = {k: v[:1].contiguous() for k, v in gpu.items() if k != "A"}
    one["A"] = gpu["A"]
    with pytest.raises(AssertionError, match="cu_seqlens must be provided"):
        mamba_chunk_scan_combined(**one, chunk_size=64, return_varlen_states=True, **kw)
    # cu_seqlens without return_varlen_states is ignored, as in the reference
    out = mamba_chunk_scan_combined(**one, chunk_size=64, cu_seqlens=cu, **kw)
    assert torch.is_tensor(out)
    x = one["x"].clone().requires_grad_(True)
    out, vst = mamba_chunk_scan_combined(**dict(one, x=x), chunk_size=64, cu_seqlens=cu,
                                         return_varlen_states=True, **kw)
    with pytest.raises(AssertionError, match="not supported in backward"):
        out.sum().backward()


def _random_ssd_cases(n, seed=4242):
    """Seeded random problems over the supported space, forward and backward."""
    rng = np.random.default_rng(seed)
    flags = ["D", "D_hdim", "z", "bias", "init", "seq", "limit", "final"]
    cases = []
    for _ in range(n):
        G = int(rng.choice([1, 2]))
        H = G * int(rng.integers(1, 4))
        opts = tuple(f for f in flags if rng.random() < 0.4)
        if "D" in opts and "D_hdim" in opts:
            opts = tuple(f for f in opts if f != "D")
        cases.append((int(rng.integers(1, 3)), int(rng.integers(1, 600)), H,
                      int(rng.choice([32, 64, 128])), G, int(rng.choice([32, 64, 128, 256])),
                      int(rng.choice([64, 128, 256])), opts,
                      [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]))
    return cases


@pytest.mark.parametrize("case", _random_ssd_cases(8), ids=lambda c: "-".join(map(str, c)).replace("torch.", ""))
def test_ssd_random_problems_forward_and_backward(case):
    batch, L, H, P, G, N, Q, opts, dtype = case
    t, kw = make(batch, L, H, P, G, N, dtype, seed=L * 3 + N, opts=opts)
    final = "final" in opts
    g = torch.Generator().manual_seed(L + 1)
    dy = torch.randn(batch, L, H, P, generator=g)
    dfin = torch.randn(batch, H, P, N, generator=g)
    names = [k for k, v in t.items() if v.is_floating_point()]
    gpu = {k: (v.to(DEV).requires_grad_(True) if k in names else v.to(DEV)) for k, v in t.items()}
    res = mamba_chunk_scan_combined(**gpu, chunk_size=Q, return_final_states=final, **kw)
    out, fin = res if final else (res, None)
    cpu = {k: (v.double().requires_grad_(True) if k in names else v) for k, v in t.items()}
    ref, _, ref_fin = ssd_chunked_ref(**cpu, chunk_size=Q, compute_dtype=torch.float64, **kw)
    check(out, ref.detach(), dtype, "out")
    loss = (out.float() * dy.to(DEV)).sum() + ((fin * dfin.to(DEV)).sum() if final else 0.0)
    loss.backward()
    rloss = (ref * dy.double()).sum() + ((ref_fin * dfin.double()).sum() if final else 0.0)
    rloss.backward()
    for k in names:
        check_grad(gpu[k].grad, cpu[k].grad, dtype, "d" + k)
