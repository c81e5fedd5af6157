"""s6_fwd_noalloc, the forward whose workspace is the library's per-device scratch array,
against s6_fwd with a caller workspace: identical kernels, so identical bits.  Two calls in
a row on the same device, the second with a smaller problem, so the second reads a scratch
array that still holds the first call's contents."""
import ctypes

import pytest
import torch

import s6scan
from s6scan import _lib
from s6scan.configs import CONFIGS, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(i, no_alloc, z=None, bias=None, softplus=False, cu=None):
    out, out_z, ck, ls = s6scan.selective_scan_forward(
        i["x"].mT, i["delta"].mT, i["A"], i["B"].mT, i["C"].mT, D=i["D"], z=z, delta_bias=bias,
        delta_softplus=softplus, cu_seqlens=cu, want_ckpt=True, want_last_state=True,
        no_alloc=no_alloc)
    torch.cuda.synchronize()
    return [t for t in (out, out_z, ck, ls) if t is not None]


def test_noalloc_forward_equals_workspace_forward_twice(monkeypatch):
    # the chunked forward is the one with a workspace (chunk summaries): force it for the
    # dense problem, which the library would otherwise run on its single-pass kernel
    monkeypatch.setenv("S6_FWD_PATH", "chunked")
    print("case: cfg1 shape (workspace ~18 MB), then a smaller varlen problem with z", flush=True)
    big = {k: v.to(DEV) for k, v in make_inputs(CONFIGS[1]).items()}
    need = _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(s6scan.selective_scan_interface._problem(
        big["x"].mT, big["B"].mT, None, big["D"], None, False,
        s6scan.check_inputs(big["x"].mT, big["delta"].mT, big["A"], big["B"].mT, big["C"].mT,
                            big["D"]))))
    assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
    ref = _run(big, False)
    got = _run(big, True)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    del big, ref, got

    small = {k: v.to(DEV) for k, v in make_inputs(CONFIGS[4], seqlen=6000, dim=192).items()}
    g = torch.Generator().manual_seed(11)
    z = torch.randn(1, small["x"].shape[1], 192, generator=g).to(torch.bfloat16).to(DEV).mT
    bias = (0.1 * torch.randn(192, generator=g)).to(DEV)
    kw = dict(z=z, bias=bias, softplus=True, cu=small["cu_seqlens"])
    ref = _run(small, False, **kw)
    got = _run(small, True, **kw)
    assert len(got) == 4
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    # and with a problem the single-pass kernel runs (no workspace at all)
    monkeypatch.setenv("S6_FWD_PATH", "lanes")
    ref = _run(small3 := {k: v[:, :512] if k in ("x", "delta", "B", "C") else v
                          for k, v in small.items() if k != "cu_seqlens"}, False)
    got = _run(small3, True)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
