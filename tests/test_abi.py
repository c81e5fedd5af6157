"""The C ABI library (libs6scan.so) without a GPU: it loads, exports every entry point that
include/*.h (s6scan.h, causal_conv1d.h) declare, and its host-only validation rejects bad
arguments with the documented error codes.  No compute call is made here."""
import glob
import ctypes
import os
import re

import pytest

from s6scan import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "s6scan.h")
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"\b(s6_[a-z_0-9]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_function():
    declared = header_functions()
    assert "s6_fwd" in declared and "s6_bwd" in declared
    assert "s6_causal_conv1d_fwd" in declared and "s6_causal_conv1d_bwd" in declared
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [f for f in declared if not hasattr(lib, f)]
    assert not missing, f"declared in include/*.h but not exported: {missing}"
    assert set(declared) == set(_lib.EXPORTS), "ctypes binding and header disagree"


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (S6_[A-Z_]+) (\d+)", text))
    assert int(consts["S6_ABI_VERSION"]) == _lib.ABI_VERSION == _lib.LIB.s6_abi_version()
    assert int(consts["S6_CKPT_INTERVAL"]) == _lib.CKPT_INTERVAL
    assert int(consts["S6_MAX_DSTATE_FWD"]) == _lib.MAX_DSTATE_FWD
    assert int(consts["S6_MAX_DSTATE_BWD"]) == _lib.MAX_DSTATE_BWD
    assert (int(consts["S6_FWD_CHUNKED"]), int(consts["S6_FWD_CHUNKED_ROWS"]),
            int(consts["S6_FWD_SINGLE_PASS"])) == (_lib.FWD_CHUNKED, _lib.FWD_CHUNKED_ROWS,
                                                   _lib.FWD_SINGLE_PASS)


def prob(**kw):
    base = dict(batch=2, dim=128, seqlen=100, dstate=16, ngroups=1, io_dtype=_lib.BF16,
                bc_dtype=_lib.BF16, has_D=1, has_z=0, has_delta_bias=0, delta_softplus=0, nseq=0)
    base.update(kw)
    return _lib.S6Problem(**base)


def validate(**kw):
    return _lib.LIB.s6_validate_problem(ctypes.byref(prob(**kw)))


def test_valid_problem():
    assert validate() == _lib.OK
    assert _lib.last_error() == ""


@pytest.mark.parametrize("kw,code,msg", [
    (dict(batch=0), _lib.E_INVALID, "must be >= 1"),
    (dict(seqlen=0), _lib.E_INVALID, "must be >= 1"),
    (dict(dim=100, ngroups=3), _lib.E_INVALID, "divisible"),
    (dict(io_dtype=7), _lib.E_INVALID, "dtype"),
    (dict(dstate=65), _lib.E_UNSUPPORTED, "dstate"),
    (dict(nseq=-1), _lib.E_INVALID, "nseq"),
    (dict(nseq=4, batch=2), _lib.E_INVALID, "batch == 1"),
])
def test_invalid_problems(kw, code, msg):
    assert validate(**kw) == code
    assert msg in _lib.last_error()


def test_num_checkpoints():
    # one entry per S6_CKPT_INTERVAL (8) steps, the last one possibly partial
    for L, want in ((1, 1), (8, 1), (9, 2), (32, 4), (33, 5), (4096, 512)):
        assert _lib.LIB.s6_num_checkpoints(ctypes.byref(prob(seqlen=L))) == want


def test_workspace_sizes_are_reported_and_grow_with_the_problem():
    small = _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(prob(seqlen=4096)))
    big = _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(prob(seqlen=4096, batch=8)))
    assert 0 < small <= big
    assert (_lib.LIB.s6_bwd_workspace_bytes(ctypes.byref(prob(seqlen=4096)))
            >= _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(prob(seqlen=4096))))
    assert _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(prob(batch=0))) == 0


def fwd_args(**kw):
    a = _lib.S6FwdArgs()
    a.p = prob(**kw)
    fake = 0x10000  # never dereferenced: validation is host-only
    for f in ("u", "delta", "A", "B", "C", "D", "out"):
        setattr(a, f, fake)
    a.u_stride = a.delta_stride = a.out_stride = (a.p.dim * a.p.seqlen, a.p.seqlen, 1)
    a.A_stride = (a.p.dstate, 1)
    a.B_stride = a.C_stride = (a.p.dstate * a.p.seqlen, a.p.dstate * a.p.seqlen, a.p.seqlen, 1)
    a.D_stride = 1
    nb = _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(a.p))
    a.workspace, a.workspace_bytes = fake, nb
    return a


def test_validate_fwd_ok_and_errors():
    a = fwd_args()
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.OK
    a.u = None
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.E_INVALID
    assert "u must not be NULL" in _lib.last_error()
    a = fwd_args(dstate=8)  # the chunked forward (the single-pass one needs no workspace)
    a.workspace_bytes = 8
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.E_WORKSPACE
    a = fwd_args()
    a.delta_stride = (1, -1, 1)
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.E_INVALID
    assert "negative stride" in _lib.last_error()
    a = fwd_args(has_z=1)
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.E_INVALID
    assert "z must not be NULL" in _lib.last_error()
    a = fwd_args(nseq=3, batch=1)
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.E_INVALID
    assert "cu_seqlens" in _lib.last_error()


def test_validate_checkpoint_strides():
    # x_ckpt strides [batch, checkpoint, dim, dstate]: all zero = contiguous; any non-negative
    # batch / checkpoint / dim strides with a unit dstate stride (the native-module layout,
    # [batch, nck, dim, 2*dstate] storage with the states in the first half, among them);
    # negative strides and strided states are rejected
    a = fwd_args()
    a.x_ckpt = 0x10000
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.OK
    nck = _lib.LIB.s6_num_checkpoints(ctypes.byref(a.p))
    N, D = a.p.dstate, a.p.dim
    a.x_ckpt_stride = (nck * D * 2 * N, D * 2 * N, 2 * N, 1)
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.OK
    a.x_ckpt_stride = (0, 0, -N, 1)
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.E_INVALID
    assert "x_ckpt has a negative stride" in _lib.last_error()
    a.x_ckpt_stride = (nck * D * 2 * N, D * 2 * N, 2 * N, 2)
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.E_UNSUPPORTED
    assert "dstate stride must be 1" in _lib.last_error()
    a.x_ckpt = None  # no checkpoints written: strides are not looked at
    a.x_ckpt_stride = (0, 0, -1, 0)
    assert _lib.LIB.s6_validate_fwd(ctypes.byref(a)) == _lib.OK


def test_validate_bwd_dstate_limits():
    def args(N):
        a = _lib.S6BwdArgs()
        a.p = prob(dstate=N)
        for f in ("u", "delta", "A", "B", "C", "D", "dout", "x_ckpt", "du", "ddelta", "dA", "dB",
                  "dC", "dD"):
            setattr(a, f, 0x10000)
        return a
    # dstate 32 and 64 are accepted (split into groups of 16); the call then stops at the
    # missing workspace, which the larger dstate makes bigger
    for N in (24, 32, 64):
        assert _lib.LIB.s6_validate_bwd(ctypes.byref(args(N))) == _lib.E_WORKSPACE
    ws = [_lib.LIB.s6_bwd_workspace_bytes(ctypes.byref(prob(dstate=N))) for N in (16, 24, 64)]
    assert ws[0] < ws[1] < ws[2]
    assert _lib.LIB.s6_validate_bwd(ctypes.byref(args(65))) == _lib.E_UNSUPPORTED


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(ImportError, match="native library not found"):
        _lib.load_library(str(tmp_path / "libs6scan.so"))


def conv_prob(**kw):
    d = dict(batch=2, dim=64, seqlen=300, width=4, io_dtype=_lib.BF16, silu=1)
    d.update(kw)
    return _lib.S6ConvProblem(**d)


def conv_args(bwd=False, **kw):
    a = _lib.S6ConvBwdArgs() if bwd else _lib.S6ConvFwdArgs()
    a.p = conv_prob(**kw)
    fake = ctypes.c_void_p(0x100000)
    a.x, a.x_stride = fake, (300 * 64, 1, 64)
    a.weight, a.weight_stride = fake, (4, 1)
    if bwd:
        a.dout, a.dout_stride = fake, (300 * 64, 1, 64)
        a.dx, a.dx_stride = fake, (300 * 64, 1, 64)
        a.dweight, a.dweight_stride = fake, (4, 1)
        a.workspace = fake
        a.workspace_bytes = _lib.LIB.s6_causal_conv1d_bwd_workspace_bytes(ctypes.byref(a.p))
    else:
        a.out, a.out_stride = fake, (300 * 64, 1, 64)
    return a


def test_conv_validate_ok_and_errors():
    LIB = _lib.LIB
    assert LIB.s6_causal_conv1d_validate_fwd(ctypes.byref(conv_args())) == _lib.OK
    assert LIB.s6_causal_conv1d_validate_bwd(ctypes.byref(conv_args(True))) == _lib.OK
    # causal_conv1d supports widths 2..4 only
    for w in (1, 5):
        assert LIB.s6_causal_conv1d_validate_fwd(ctypes.byref(conv_args(width=w))) == _lib.E_UNSUPPORTED
        assert "width" in _lib.last_error()
    assert LIB.s6_causal_conv1d_validate_fwd(ctypes.byref(conv_args(seqlen=0))) == _lib.E_INVALID
    assert LIB.s6_causal_conv1d_validate_fwd(ctypes.byref(conv_args(io_dtype=7))) == _lib.E_INVALID
    a = conv_args()
    a.out = None
    assert LIB.s6_causal_conv1d_validate_fwd(ctypes.byref(a)) == _lib.E_INVALID
    assert "out" in _lib.last_error()
    a = conv_args(True)
    a.workspace_bytes -= 4
    assert LIB.s6_causal_conv1d_validate_bwd(ctypes.byref(a)) == _lib.E_WORKSPACE
    a = conv_args(True)
    a.dx_stride = (300 * 64, -1, 64)
    assert LIB.s6_causal_conv1d_validate_bwd(ctypes.byref(a)) == _lib.E_INVALID


def test_conv_workspace_holds_one_partial_row_per_block():
    LIB = _lib.LIB
    row = 64 * 5 * 4  # dim * (width + 1) fp32 partial sums
    small = LIB.s6_causal_conv1d_bwd_workspace_bytes(ctypes.byref(conv_prob(seqlen=256)))
    assert small == 2 * row + row  # one partial row per batch row + one slice row
    big = LIB.s6_causal_conv1d_bwd_workspace_bytes(ctypes.byref(conv_prob(seqlen=1 << 16)))
    assert small < big <= 2 * 256 * row + 256 + 64 * row
    assert LIB.s6_causal_conv1d_bwd_workspace_bytes(ctypes.byref(conv_prob(width=9))) == 0


def _validate_cu(values, seqlen):
    arr = (ctypes.c_int32 * len(values))(*values)
    return _lib.LIB.s6_validate_cu_seqlens(ctypes.cast(arr, ctypes.c_void_p), len(values) - 1,
                                           seqlen)


@pytest.mark.parametrize("values,msg", [
    ([10, 100], "cu_seqlens[0] must be 0"),                # does not start at 0
    ([0, 60, 50, 100], "non-decreasing"),                  # not monotone
    ([0, 50], "must equal seqlen 100"),                    # does not end at seqlen
    ([0, 100, 120], "must equal seqlen 100"),              # runs past the end
    ([0, -5, 100], "non-decreasing"),
    ([0], "nseq"),                                         # no sequence
])
def test_cu_seqlens_validator_rejects(values, msg):
    """Host-only check of packed-varlen offsets (the reference's varlen convention,
    ssd_combined.py:576-577): malformed vectors return S6_E_INVALID and are never launched."""
    assert _validate_cu(values, 100) == _lib.E_INVALID
    assert msg in _lib.last_error()


@pytest.mark.parametrize("values", [[0, 100], [0, 0, 100], [0, 40, 40, 100, 100], [0, 1, 2, 100]])
def test_cu_seqlens_validator_accepts(values):
    # empty sequences (repeated offsets) are allowed, as in the reference's seq_idx form
    assert _validate_cu(values, 100) == _lib.OK
    assert _lib.last_error() == ""


def test_cu_seqlens_validator_null():
    assert _lib.LIB.s6_validate_cu_seqlens(None, 1, 100) == _lib.E_INVALID


def test_noalloc_forward_rejects_problems_above_its_scratch():
    """s6_fwd_noalloc checks the problem's workspace against its fixed per-device scratch on
    the host and refuses before any device work (so this runs without a GPU; the pointers
    are never dereferenced)."""
    batch, dim, L, N = 64, 256, 65536, 8      # dstate 8: the chunked forward (workspace)
    p = _lib.S6Problem(batch, dim, L, N, 1, _lib.BF16, _lib.BF16, 1, 0, 0, 0, 0)
    a = _lib.S6FwdArgs()
    a.p = p
    fake = ctypes.c_void_p(256)
    a.u = a.delta = a.A = a.B = a.C = a.D = a.out = fake
    a.u_stride = a.delta_stride = a.out_stride = (dim * L, L, 1)
    a.A_stride = (N, 1)
    a.B_stride = a.C_stride = (N * L, N * L, L, 1)      # L-contiguous rows: relaid out
    a.D_stride = 1
    need = _lib.LIB.s6_fwd_workspace_bytes(ctypes.byref(p))
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    assert _lib.LIB.s6_fwd_noalloc(ctypes.byref(a), None) == _lib.E_WORKSPACE
    assert "scratch" in _lib.last_error()
    # argument errors are reported as by s6_fwd
    a.u = None
    assert _lib.LIB.s6_fwd_noalloc(ctypes.byref(a), None) == _lib.E_INVALID


def test_forward_kernel_choice(monkeypatch):
    """s6_fwd_single_pass names the kernel s6_fwd will run: the single-pass kernel for dense
    batches with enough (channel, state) lanes and no z gate, the chunked kernels otherwise
    (varlen, small problems, dstate <= 8, the z gate); S6_FWD_PATH forces either."""
    monkeypatch.delenv("S6_FWD_PATH", raising=False)
    q = lambda **kw: _lib.LIB.s6_fwd_single_pass(ctypes.byref(prob(**kw)))
    big = dict(batch=32, dim=256, seqlen=4096, dstate=16)
    assert q(**big) == 1
    assert q(**big, has_z=1) == 0
    assert q(**dict(big, dstate=8)) == 0
    assert q(batch=1, dim=256, seqlen=4096, dstate=16) == 0          # 64 waves
    assert q(batch=1, dim=1024, seqlen=4096, dstate=16, nseq=3) == 0  # varlen
    monkeypatch.setenv("S6_FWD_PATH", "lanes")
    assert q(batch=1, dim=256, seqlen=4096, dstate=16) == 1
    assert q(batch=1, dim=1024, seqlen=4096, dstate=16, nseq=3) == 0  # never varlen
    monkeypatch.setenv("S6_FWD_PATH", "chunked")
    assert q(**big) == 0
    assert q(batch=0) == _lib.E_INVALID


def test_forward_kernel_for_arguments(monkeypatch):
    """s6_fwd_kernel names the forward kernels for a call's arguments.  The chunked kernels
    move u / delta / z / out / out_z in whole 8-step row blocks only for a contiguous time axis
    with 16-byte aligned rows and blocks, seqlen a multiple of 8 and dstate <= 32; on an
    L-contiguous layout every single-pass-eligible problem (dstate 9-64, no varlen) takes the
    single-pass kernel, z gate and small wave counts included.  Overrides S6_FWD_ROWVEC=0 and
    S6_FWD_PATH.  Host-only (fake pointers)."""
    CH, ROWS, SP = _lib.FWD_CHUNKED, _lib.FWD_CHUNKED_ROWS, _lib.FWD_SINGLE_PASS
    monkeypatch.delenv("S6_FWD_ROWVEC", raising=False)
    monkeypatch.delenv("S6_FWD_PATH", raising=False)
    q = lambda a: _lib.LIB.s6_fwd_kernel(ctypes.byref(a))
    assert q(fwd_args(seqlen=1024)) == SP                      # [B, D, L] L-contiguous
    assert q(fwd_args(seqlen=1024, dstate=8)) == ROWS          # below the single-pass range
    assert q(fwd_args(seqlen=1004, dstate=8)) == CH            # a partial last block
    zl = fwd_args(seqlen=1024, has_z=1)
    zl.z = zl.out_z = 0x20000
    zl.z_stride = zl.out_z_stride = zl.u_stride
    assert q(zl) == SP                                         # the z gate too, on this layout
    cl = fwd_args(seqlen=1024)
    cl.u_stride = cl.delta_stride = cl.out_stride = (cl.p.dim * 1024, 1, cl.p.dim)
    assert q(cl) == CH                                         # channel-last, 16 waves
    big = fwd_args(batch=32, dim=256, seqlen=4096)
    big.u_stride = big.delta_stride = big.out_stride = (256 * 4096, 1, 256)
    assert q(big) == SP                                        # channel-last, 2048 waves
    monkeypatch.setenv("S6_FWD_PATH", "chunked")
    assert q(fwd_args(seqlen=1024)) == ROWS
    assert q(fwd_args(seqlen=1000)) == ROWS                    # 1000 = 125 blocks of 8
    assert q(fwd_args(seqlen=1004)) == CH
    assert q(fwd_args(seqlen=1024, dstate=32)) == ROWS
    assert q(fwd_args(seqlen=1024, dstate=48)) == CH           # one wave per 16 states
    a = fwd_args(seqlen=1024)
    a.u_stride = (a.p.dim * 1024, 1, a.p.dim)                  # one channel-last view
    assert q(a) == CH
    a = fwd_args(seqlen=1024)
    a.out = 0x10000 + 8                                        # out rows 8-byte aligned only
    assert q(a) == CH
    a = fwd_args(seqlen=1024, io_dtype=_lib.F32, bc_dtype=_lib.F32)
    a.delta_stride = (a.p.dim * 1026, 1026, 1)                 # rows 4104 B apart: not 16-aligned
    assert q(a) == CH
    a = fwd_args(seqlen=1024, has_z=1)
    assert q(a) == _lib.E_INVALID                              # z / out_z missing
    a.z = a.out_z = 0x20000
    a.z_stride = a.out_z_stride = a.u_stride
    assert q(a) == ROWS
    a.out_z_stride = (a.p.dim * 1024, 1, a.p.dim)
    assert q(a) == CH
    monkeypatch.setenv("S6_FWD_ROWVEC", "0")
    assert q(fwd_args(seqlen=1024)) == CH


def test_backward_row_block_choice(monkeypatch):
    """s6_bwd_row_blocks: the backward's row blocks need every per-channel tensor it reads
    and writes L-contiguous and 16-byte aligned, seqlen a multiple of 8 and dstate <= 16;
    S6_BWD_ROWVEC=0 turns them off.  Host-only (fake pointers)."""
    monkeypatch.delenv("S6_BWD_ROWVEC", raising=False)

    def args(L=1024, N=16, z=0):
        a = _lib.S6BwdArgs()
        a.p = prob(seqlen=L, dstate=N, has_z=z)
        rows = ("u", "delta", "dout", "du", "ddelta") + (("z", "out", "dz") if z else ())
        for f in rows:
            setattr(a, f, 0x10000)
            setattr(a, f + "_stride", (a.p.dim * L, L, 1))
        return a

    q = lambda a: _lib.LIB.s6_bwd_row_blocks(ctypes.byref(a))
    assert q(args()) == 1
    assert q(args(z=1)) == 1
    assert q(args(L=1004)) == 0
    assert q(args(N=24)) == 0                                   # state groups of 16
    a = args(z=1)
    a.dz_stride = (a.p.dim * 1024, 1, a.p.dim)                  # a channel-last output
    assert q(a) == 0
    a = args(z=1)
    a.out_z, a.out_z_stride = 0x10008, a.u_stride               # out_z 8-byte aligned only
    assert q(a) == 0
    a = args()
    a.ddelta = 0x10004
    assert q(a) == 0
    monkeypatch.setenv("S6_BWD_ROWVEC", "0")
    assert q(args()) == 0
    assert q(args(L=0)) == _lib.E_INVALID


def _ssd_problem(P=64, N=32, Q=64, z=0, L=300, H=4, G=2, batch=2):
    return _lib.S6SsdProblem(batch, L, H, P, G, N, Q, _lib.BF16, 1, 0, z, 1, 1, 0, 0, 0.0,
                             float("inf"))


@pytest.mark.parametrize("shape", [(160, 32, 64), (0, 32, 64), (64, 300, 64), (64, 0, 64),
                                   (64, 32, 32), (64, 32, 100), (64, 32, 320)])
def test_ssd_shape_limits_rejected(shape):
    """headdim above 128, dstate above 256 and chunk sizes that are not 64, 128, 192 or 256
    have no kernel: the workspace query says so (0) before any launch."""
    P, N, Q = shape
    assert _lib.LIB.s6_ssd_fwd_workspace_bytes(ctypes.byref(_ssd_problem(P, N, Q))) == 0
    assert _lib.LIB.s6_ssd_bwd_workspace_bytes(ctypes.byref(_ssd_problem(P, N, Q))) == 0


@pytest.mark.parametrize("z", [0, 1])
def test_ssd_padded_shapes_accepted_with_staging_buffers(z):
    """Shapes off the kernels' tiles (zoology Mamba-2's d_state 8 / 16 / 24, headdim 48,
    chunk 192) are accepted; their workspace is the next tile shape's plus the zero-padded
    copies: B and C at dstate 24 (-> 32), and x, out (z, out_x) at headdim 48 (-> 64), plus
    dout, dx (dz) in the backward."""
    ws = lambda f, *a, **k: getattr(_lib.LIB, f)(ctypes.byref(_ssd_problem(*a, z=z, **k)))
    al = lambda n: (n + 255) // 256 * 256
    batch, L, H, G = 2, 300, 4, 2
    for f in ("s6_ssd_fwd_workspace_bytes", "s6_ssd_bwd_workspace_bytes"):
        assert ws(f, 64, 32, 192) > 0
        for N in (8, 16, 24):
            assert ws(f, 64, N, 256) == ws(f, 64, 32, 256) + 2 * al(batch * L * G * 32 * 2)
    nP = 2 + 2 * z  # x, out (, z, out_x)
    assert (ws("s6_ssd_fwd_workspace_bytes", 48, 32, 64)
            == ws("s6_ssd_fwd_workspace_bytes", 64, 32, 64) + nP * al(batch * L * H * 64 * 2))
    nPb = nP + 2 + z  # + dout, dx (, dz)
    assert (ws("s6_ssd_bwd_workspace_bytes", 48, 32, 64)
            == ws("s6_ssd_bwd_workspace_bytes", 64, 32, 64) + nPb * al(batch * L * H * 64 * 2))
