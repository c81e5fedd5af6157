"""The five benchmark/parity workloads of the S6 scan and their synthetic inputs.

Distributions and seeds are the ones fixed for this path; the draw order is this module's
convention (documented so any run can regenerate the same tensors):

    g = torch.Generator("cpu").manual_seed(seed)
    # varlen config only, drawn first:
    lengths = randint(128, 8193, (nseq,)); T = sum; cu_seqlens = [0, cumsum]; B = 1, L = T
    x = randn(B,L,D); dtr = randn(B,L,D); Au = rand(D,N); Bt = randn(B,L,N); Ct = randn(B,L,N)
    Dskip = randn(D);  dy = randn(B,L,D)                       (backward configs only)
    delta = softplus(0.5 * dtr + shift)   (shift -1, or -3 for the slow-decay config)
    A = -exp(Au * ln 16)                  (fp32)
    16-bit configs cast x, delta, Bt, Ct, dy after generation; A and Dskip stay fp32.

The scan is called on channel-last views, as a [B, L, D] producer would:
    selective_scan_fn(x.mT, delta.mT, A, Bt.mT, Ct.mT, D=Dskip, return_last_state=True)
"""
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class ScanConfig:
    name: str
    batch: int
    seqlen: int
    dim: int
    dstate: int
    dtype: torch.dtype
    seed: int
    shift: float = -1.0
    backward: bool = False
    nseq: int = 0          # > 0: packed varlen with nseq sequences of length U[128, 8192]

    def algorithmic_bytes(self, seqlen=None, with_backward=None):
        """Bytes that must cross HBM once per call, each tensor counted once (dB and dC at
        the input width, as the headline figures count them)."""
        L = self.seqlen if seqlen is None else seqlen
        io = 2 if self.dtype in (torch.bfloat16, torch.float16) else 4
        B, D, N = self.batch, self.dim, self.dstate
        nls = self.nseq if self.nseq else B
        fwd = B * L * D * 3 * io + B * L * N * 2 * io + 4 * D * N + 4 * D + 4 * nls * D * N
        if self.nseq:
            fwd += 4 * (self.nseq + 1)
        bwd_on = self.backward if with_backward is None else with_backward
        if not bwd_on:
            return fwd
        bwd = B * L * D * 5 * io + B * L * N * 4 * io + 2 * (4 * D * N + 4 * D)
        return fwd + bwd


CONFIGS = {
    0: ScanConfig("cfg0_fp32_B1_L1024_D128_N16", 1, 1024, 128, 16, torch.float32, 0),
    1: ScanConfig("cfg1_bf16_B32_L4096_D256_N16", 32, 4096, 256, 16, torch.bfloat16, 1),
    2: ScanConfig("cfg2_fp32_B16_L16384_D256_N64_slow", 16, 16384, 256, 64, torch.float32, 2,
                  shift=-3.0),
    3: ScanConfig("cfg3_bf16_B8_L8192_D768_N16_fwdbwd", 8, 8192, 768, 16, torch.bfloat16, 3,
                  backward=True),
    4: ScanConfig("cfg4_bf16_varlen64_D1024_N16_fwdbwd", 1, 0, 1024, 16, torch.bfloat16, 4,
                  backward=True, nseq=64),
}


def make_inputs(cfg: ScanConfig, device="cpu", seqlen=None, batch=None, dim=None):
    """Synthetic inputs of ``cfg`` (optionally shrunk).  Returns a dict with x, delta, A, B,
    C, D (and dy for backward configs, cu_seqlens for varlen) in [B, L, *] layout."""
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    res = {}
    B = cfg.batch if batch is None else batch
    D = cfg.dim if dim is None else dim
    N = cfg.dstate
    if cfg.nseq:
        lengths = torch.randint(128, 8193, (cfg.nseq,), generator=g)
        if seqlen is not None:  # shrink every sequence proportionally (tests)
            lengths = torch.clamp((lengths * seqlen) // int(lengths.sum()), min=1)
        cu = torch.zeros(cfg.nseq + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(lengths, 0).to(torch.int32)
        L = int(cu[-1])
        res["cu_seqlens"] = cu
        B = 1
    else:
        L = cfg.seqlen if seqlen is None else seqlen
    x = torch.randn(B, L, D, generator=g)
    dtr = torch.randn(B, L, D, generator=g)
    Au = torch.rand(D, N, generator=g)
    Bt = torch.randn(B, L, N, generator=g)
    Ct = torch.randn(B, L, N, generator=g)
    Dsk = torch.randn(D, generator=g)
    dy = torch.randn(B, L, D, generator=g) if cfg.backward else None
    delta = F.softplus(0.5 * dtr + cfg.shift)
    A = -torch.exp(Au * math.log(16.0))
    dt = cfg.dtype
    res.update(x=x.to(dt), delta=delta.to(dt), A=A, B=Bt.to(dt), C=Ct.to(dt), D=Dsk)
    if dy is not None:
        res["dy"] = dy.to(dt)
    if device != "cpu":
        res = {k: v.to(device) for k, v in res.items()}
    return res
