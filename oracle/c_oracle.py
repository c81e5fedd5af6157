"""ctypes wrapper of oracle/s6_oracle.c -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this, as the
checker.  Inputs are torch CPU tensors in the reference's logical layout (u/delta/z/dout
[B, D, L], A [D, N], B/C [B, N, L] or [B, G, N, L]); they are upcast to fp32 and made
dense before the call.  Outputs are fp32 (the caller casts ``out`` to the input dtype,
as selective_scan_interface.py:156 does).
"""
import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libs6oracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = ctypes.CDLL(_SO)
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        _lib.s6o_fwd.argtypes = [i64] * 5 + [vp] * 8 + [ctypes.c_int, vp, ctypes.c_int32, vp, vp]
        _lib.s6o_bwd.argtypes = ([i64] * 5 + [vp] * 8 + [ctypes.c_int, vp, ctypes.c_int32]
                                 + [vp] * 9)
        _lib.s6o_fwd64.argtypes = _lib.s6o_fwd.argtypes
        _lib.s6o_fwd.restype = None
        _lib.s6o_fwd64.restype = None
        _lib.s6o_bwd.restype = None
    return _lib


def _f(t):
    return None if t is None else t.detach().to(torch.float32).contiguous()


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _bc4(M):
    M = _f(M)
    return M.unsqueeze(1).contiguous() if M.dim() == 3 else M


def set_threads(n):
    os.environ["OMP_NUM_THREADS"] = str(n)


def fwd(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
        cu_seqlens=None):
    """Returns (out fp32 [B, D, L], last_state fp32 [B|nseq, D, N])."""
    lib = _load()
    uu, dl, AA, BB, CC = _f(u), _f(delta), _f(A), _bc4(B), _bc4(C)
    Dv, zz, bb = _f(D), _f(z), _f(delta_bias)
    Bsz, Dm, L = uu.shape
    N, G = AA.shape[1], BB.shape[1]
    cu = None if cu_seqlens is None else cu_seqlens.to(torch.int32).contiguous()
    nseq = 0 if cu is None else cu.numel() - 1
    out = torch.empty(Bsz, Dm, L, dtype=torch.float32)
    ls = torch.empty(nseq if nseq else Bsz, Dm, N, dtype=torch.float32)
    lib.s6o_fwd(Bsz, Dm, L, N, G, _p(uu), _p(dl), _p(AA), _p(BB), _p(CC), _p(Dv), _p(zz),
                _p(bb), int(bool(delta_softplus)), _p(cu), nseq, _p(out), _p(ls))
    return out, ls


def fwd64(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
          cu_seqlens=None):
    """The recurrence in float64 from the fp32-cast inputs: (out, last_state) as float64
    tensors -- the exact value that fp32 results are measured against."""
    lib = _load()
    uu, dl, AA, BB, CC = _f(u), _f(delta), _f(A), _bc4(B), _bc4(C)
    Dv, zz, bb = _f(D), _f(z), _f(delta_bias)
    Bsz, Dm, L = uu.shape
    N, G = AA.shape[1], BB.shape[1]
    cu = None if cu_seqlens is None else cu_seqlens.to(torch.int32).contiguous()
    nseq = 0 if cu is None else cu.numel() - 1
    out = torch.empty(Bsz, Dm, L, dtype=torch.float64)
    ls = torch.empty(nseq if nseq else Bsz, Dm, N, dtype=torch.float64)
    lib.s6o_fwd64(Bsz, Dm, L, N, G, _p(uu), _p(dl), _p(AA), _p(BB), _p(CC), _p(Dv), _p(zz),
                  _p(bb), int(bool(delta_softplus)), _p(cu), nseq, _p(out), _p(ls))
    return out, ls


def bwd(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None, delta_softplus=False,
        cu_seqlens=None):
    """Returns dict du, ddelta, dA, dB, dC, dD, dz, ddelta_bias (fp32; dB/dC in B/C's rank)."""
    lib = _load()
    uu, dl, AA, BB, CC, do = _f(u), _f(delta), _f(A), _bc4(B), _bc4(C), _f(dout)
    Dv, zz, bb = _f(D), _f(z), _f(delta_bias)
    Bsz, Dm, L = uu.shape
    N, G = AA.shape[1], BB.shape[1]
    cu = None if cu_seqlens is None else cu_seqlens.to(torch.int32).contiguous()
    nseq = 0 if cu is None else cu.numel() - 1
    du = torch.empty_like(uu)
    ddl = torch.empty_like(uu)
    dA = torch.empty_like(AA)
    dB = torch.empty_like(BB)
    dC = torch.empty_like(CC)
    dD = torch.empty(Dm) if D is not None else None
    dz = torch.empty_like(uu) if z is not None else None
    dbias = torch.empty(Dm) if delta_bias is not None else None
    lib.s6o_bwd(Bsz, Dm, L, N, G, _p(uu), _p(dl), _p(AA), _p(BB), _p(CC), _p(Dv), _p(zz),
                _p(bb), int(bool(delta_softplus)), _p(cu), nseq, _p(do), _p(du), _p(ddl),
                _p(dA), _p(dB), _p(dC), _p(dD), _p(dz), _p(dbias))
    if B.dim() == 3:
        dB = dB.squeeze(1)
    if C.dim() == 3:
        dC = dC.squeeze(1)
    return dict(du=du, ddelta=ddl, dA=dA, dB=dB, dC=dC, dD=dD, dz=dz, ddelta_bias=dbias)
