"""Regenerate tests/golden/s6_golden.npz.

The reference holds no golden vectors for the S6 scan, so these fixtures are computed by
the float64 brute force in oracle/brute64.py (itself pinned against the torch restatement
of selective_scan_ref, gradcheck and closed forms in tests/test_oracle.py).  Inputs are
stored as float32 (bf16 cases store the bf16-rounded values), outputs as float64.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle.brute64 import scan_bwd64, scan_fwd64  # noqa: E402

CASES = {
    # name: (B, L, D, N, G, dtype, z, bias+softplus, cu_seqlens, backward)
    "fp32_dense": (2, 70, 80, 16, 1, "fp32", False, False, None, True),
    "fp32_groups_z_bias": (2, 40, 128, 8, 2, "fp32", True, True, None, True),
    "bf16_dense": (1, 130, 64, 16, 1, "bf16", False, False, None, True),
    "fp32_varlen": (1, 200, 64, 16, 1, "fp32", True, True, [0, 37, 38, 150, 200], True),
    "fp32_n64": (1, 50, 64, 64, 1, "fp32", False, False, None, True),
    "fp32_n12": (2, 33, 64, 12, 1, "fp32", True, False, None, True),
    "fp32_n24_varlen": (1, 90, 64, 24, 1, "fp32", True, True, [0, 30, 31, 90], True),
}


def make_case(name, spec, seed):
    B, L, D, N, G, dt, has_z, has_bias, cu, bwd = spec
    g = torch.Generator("cpu").manual_seed(seed)
    u = torch.randn(B, D, L, generator=g)
    dl = torch.nn.functional.softplus(0.5 * torch.randn(B, D, L, generator=g) - 1.0)
    if has_bias:  # raw delta before bias + softplus
        dl = 0.5 * torch.randn(B, D, L, generator=g) - 1.0
    A = -torch.exp(torch.rand(D, N, generator=g) * np.log(16.0))
    Bm = torch.randn(B, G, N, L, generator=g)
    Cm = torch.randn(B, G, N, L, generator=g)
    Dv = torch.randn(D, generator=g)
    z = torch.randn(B, D, L, generator=g) if has_z else None
    bias = 0.3 * torch.randn(D, generator=g) if has_bias else None
    dout = torch.randn(B, D, L, generator=g)
    if dt == "bf16":
        u, dl, Bm, Cm, dout = (t.bfloat16().float() for t in (u, dl, Bm, Cm, dout))
        if z is not None:
            z = z.bfloat16().float()
    if G == 1:
        Bm, Cm = Bm[:, 0], Cm[:, 0]
    cu_np = None if cu is None else np.asarray(cu, dtype=np.int32)
    n = lambda t: None if t is None else t.numpy().astype(np.float64)
    f = scan_fwd64(n(u), n(dl), n(A), n(Bm), n(Cm), n(Dv), n(z), n(bias), has_bias, cu_seqlens=cu_np)
    out = {f"{name}/u": u, f"{name}/delta": dl, f"{name}/A": A, f"{name}/B": Bm, f"{name}/C": Cm,
           f"{name}/D": Dv, f"{name}/dout": dout}
    out = {k: v.numpy().astype(np.float32) for k, v in out.items()}
    if z is not None:
        out[f"{name}/z"] = z.numpy().astype(np.float32)
    if bias is not None:
        out[f"{name}/delta_bias"] = bias.numpy().astype(np.float32)
    if cu_np is not None:
        out[f"{name}/cu_seqlens"] = cu_np
    out[f"{name}/ref_out"] = f["out"]
    out[f"{name}/ref_last_state"] = f["last_state"]
    if bwd:
        gr = scan_bwd64(n(u), n(dl), n(A), n(Bm), n(Cm), n(dout), n(Dv), n(z), n(bias), has_bias,
                        cu_seqlens=cu_np)
        for k, v in gr.items():
            if v is not None and k != "out":
                out[f"{name}/ref_{k}"] = v
    return out


def main():
    arrays = {}
    for i, (name, spec) in enumerate(CASES.items()):
        arrays.update(make_case(name, spec, 1000 + i))
    path = os.path.join(HERE, "s6_golden.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
