"""ctypes binding of the s6scan C ABI (``include/s6scan.h``, ``include/causal_conv1d.h``,
``include/selective_state_update.h``, ``include/ssd.h``).

The shared library is built in-tree (``ml-experiments_amd/build.py``) next to this file.
There is no fallback: if the library is missing or was built for another ABI version,
importing ``s6scan`` raises ``ImportError``.

torch is imported first on purpose: torch bundles its own HIP runtime
(``libamdhip64.so.7``), and loading it before this library makes the dynamic linker bind
the library's HIP calls to that same runtime, so torch's device pointers and streams are
the ones the kernels see.
"""
import ctypes
import os

import torch  # noqa: F401  (see module docstring: must precede the HIP library)

ABI_VERSION = 6
CKPT_INTERVAL = 8
MAX_DSTATE_FWD = 64
MAX_DSTATE_BWD = 64
NOALLOC_SCRATCH_BYTES = 64 << 20

F32, BF16, F16 = 0, 1, 2
OK, E_INVALID, E_UNSUPPORTED, E_WORKSPACE, E_HIP = 0, -1, -2, -3, -4
FWD_CHUNKED, FWD_CHUNKED_ROWS, FWD_SINGLE_PASS = 0, 1, 2  # s6_fwd_kernel

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libs6scan.so")

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p


def _a(n):
    return _i64 * n


class S6Problem(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("dim", _i64), ("seqlen", _i64), ("dstate", _i64), ("ngroups", _i64),
        ("io_dtype", _i32), ("bc_dtype", _i32),
        ("has_D", _i32), ("has_z", _i32), ("has_delta_bias", _i32), ("delta_softplus", _i32),
        ("nseq", _i32),
    ]


class S6FwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", S6Problem),
        ("u", _vp), ("u_stride", _a(3)),
        ("delta", _vp), ("delta_stride", _a(3)),
        ("A", _vp), ("A_stride", _a(2)),
        ("B", _vp), ("B_stride", _a(4)),
        ("C", _vp), ("C_stride", _a(4)),
        ("D", _vp), ("D_stride", _i64),
        ("z", _vp), ("z_stride", _a(3)),
        ("delta_bias", _vp), ("delta_bias_stride", _i64),
        ("cu_seqlens", _vp),
        ("out", _vp), ("out_stride", _a(3)),
        ("out_z", _vp), ("out_z_stride", _a(3)),
        ("x_ckpt", _vp), ("x_ckpt_stride", _a(4)),
        ("last_state", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("kernel_events", _vp * 2),
    ]


class S6BwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", S6Problem),
        ("u", _vp), ("u_stride", _a(3)),
        ("delta", _vp), ("delta_stride", _a(3)),
        ("A", _vp), ("A_stride", _a(2)),
        ("B", _vp), ("B_stride", _a(4)),
        ("C", _vp), ("C_stride", _a(4)),
        ("D", _vp), ("D_stride", _i64),
        ("z", _vp), ("z_stride", _a(3)),
        ("delta_bias", _vp), ("delta_bias_stride", _i64),
        ("cu_seqlens", _vp),
        ("dout", _vp), ("dout_stride", _a(3)),
        ("x_ckpt", _vp), ("x_ckpt_stride", _a(4)),
        ("out", _vp), ("out_stride", _a(3)),
        ("du", _vp), ("du_stride", _a(3)),
        ("ddelta", _vp), ("ddelta_stride", _a(3)),
        ("dA", _vp), ("dA_stride", _a(2)),
        ("dB", _vp), ("dB_stride", _a(4)),
        ("dC", _vp), ("dC_stride", _a(4)),
        ("dD", _vp), ("dD_stride", _i64),
        ("dz", _vp), ("dz_stride", _a(3)),
        ("out_z", _vp), ("out_z_stride", _a(3)),
        ("ddelta_bias", _vp), ("ddelta_bias_stride", _i64),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("kernel_events", _vp * 2),
    ]


class S6ConvProblem(ctypes.Structure):
    _fields_ = [("batch", _i64), ("dim", _i64), ("seqlen", _i64), ("width", _i64),
                ("io_dtype", _i32), ("silu", _i32)]


class S6ConvFwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", S6ConvProblem),
        ("x", _vp), ("x_stride", _a(3)),
        ("weight", _vp), ("weight_stride", _a(2)),
        ("bias", _vp), ("bias_stride", _i64),
        ("out", _vp), ("out_stride", _a(3)),
    ]


class S6ConvBwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", S6ConvProblem),
        ("x", _vp), ("x_stride", _a(3)),
        ("weight", _vp), ("weight_stride", _a(2)),
        ("bias", _vp), ("bias_stride", _i64),
        ("dout", _vp), ("dout_stride", _a(3)),
        ("dx", _vp), ("dx_stride", _a(3)),
        ("dweight", _vp), ("dweight_stride", _a(2)),
        ("dbias", _vp), ("dbias_stride", _i64),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


class S6StateUpdateArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("nheads", _i64), ("dim", _i64), ("dstate", _i64), ("ngroups", _i64),
        ("state_dtype", _i32), ("io_dtype", _i32), ("bc_dtype", _i32),
        ("has_D", _i32), ("has_z", _i32), ("has_dt_bias", _i32), ("dt_softplus", _i32),
        ("state", _vp), ("state_stride", _a(4)),
        ("x", _vp), ("x_stride", _a(3)),
        ("dt", _vp), ("dt_stride", _a(3)),
        ("dt_bias", _vp), ("dt_bias_stride", _a(2)),
        ("A", _vp), ("A_stride", _a(3)),
        ("B", _vp), ("B_stride", _a(3)),
        ("C", _vp), ("C_stride", _a(3)),
        ("D", _vp), ("D_stride", _a(2)),
        ("z", _vp), ("z_stride", _a(3)),
        ("out", _vp), ("out_stride", _a(3)),
    ]


class S6SsdProblem(ctypes.Structure):
    _fields_ = [("batch", _i64), ("seqlen", _i64), ("nheads", _i64), ("headdim", _i64),
                ("ngroups", _i64), ("dstate", _i64), ("chunk_size", _i64),
                ("io_dtype", _i32), ("has_D", _i32), ("D_has_hdim", _i32), ("has_z", _i32),
                ("has_dt_bias", _i32), ("dt_softplus", _i32), ("has_initial_states", _i32),
                ("has_seq_idx", _i32), ("dt_min", ctypes.c_float), ("dt_max", ctypes.c_float)]


class S6SsdFwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", S6SsdProblem),
        ("x", _vp), ("x_stride", _a(4)),
        ("dt", _vp), ("dt_stride", _a(3)),
        ("A", _vp), ("A_stride", _i64),
        ("B", _vp), ("B_stride", _a(4)),
        ("C", _vp), ("C_stride", _a(4)),
        ("D", _vp), ("D_stride", _a(2)),
        ("z", _vp), ("z_stride", _a(4)),
        ("dt_bias", _vp), ("dt_bias_stride", _i64),
        ("initial_states", _vp), ("initial_states_stride", _a(4)),
        ("seq_idx", _vp), ("seq_idx_stride", _a(2)),
        ("out", _vp), ("out_stride", _a(4)),
        ("out_x", _vp), ("out_x_stride", _a(4)),
        ("final_states", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("kernel_events", _vp * 2),
        ("cu_seqlens", _vp), ("nseq", _i64),
        ("varlen_states", _vp),
    ]


class S6SsdBwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", S6SsdProblem),
        ("x", _vp), ("x_stride", _a(4)),
        ("dt", _vp), ("dt_stride", _a(3)),
        ("A", _vp), ("A_stride", _i64),
        ("B", _vp), ("B_stride", _a(4)),
        ("C", _vp), ("C_stride", _a(4)),
        ("D", _vp), ("D_stride", _a(2)),
        ("z", _vp), ("z_stride", _a(4)),
        ("dt_bias", _vp), ("dt_bias_stride", _i64),
        ("initial_states", _vp), ("initial_states_stride", _a(4)),
        ("seq_idx", _vp), ("seq_idx_stride", _a(2)),
        ("dout", _vp), ("dout_stride", _a(4)),
        ("out_x", _vp), ("out_x_stride", _a(4)),
        ("dfinal_states", _vp), ("dfinal_states_stride", _a(4)),
        ("dx", _vp), ("dx_stride", _a(4)),
        ("ddt", _vp), ("ddt_stride", _a(3)),
        ("dA", _vp),
        ("dB", _vp), ("dB_stride", _a(4)),
        ("dC", _vp), ("dC_stride", _a(4)),
        ("dD", _vp),
        ("dz", _vp), ("dz_stride", _a(4)),
        ("ddt_bias", _vp),
        ("dinitial_states", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


EXPORTS = {
    "s6_abi_version": (ctypes.c_int, []),
    "s6_last_error": (ctypes.c_char_p, []),
    "s6_validate_problem": (ctypes.c_int, [ctypes.POINTER(S6Problem)]),
    "s6_validate_fwd": (ctypes.c_int, [ctypes.POINTER(S6FwdArgs)]),
    "s6_validate_bwd": (ctypes.c_int, [ctypes.POINTER(S6BwdArgs)]),
    "s6_validate_cu_seqlens": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]),
    "s6_fwd_single_pass": (ctypes.c_int, [ctypes.POINTER(S6Problem)]),
    "s6_fwd_kernel": (ctypes.c_int, [ctypes.POINTER(S6FwdArgs)]),
    "s6_bwd_row_blocks": (ctypes.c_int, [ctypes.POINTER(S6BwdArgs)]),
    "s6_num_checkpoints": (ctypes.c_int64, [ctypes.POINTER(S6Problem)]),
    "s6_fwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(S6Problem)]),
    "s6_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(S6Problem)]),
    "s6_fwd": (ctypes.c_int, [ctypes.POINTER(S6FwdArgs), ctypes.c_void_p]),
    "s6_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(S6FwdArgs), ctypes.c_void_p]),
    "s6_bwd": (ctypes.c_int, [ctypes.POINTER(S6BwdArgs), ctypes.c_void_p]),
    "s6_causal_conv1d_validate_fwd": (ctypes.c_int, [ctypes.POINTER(S6ConvFwdArgs)]),
    "s6_causal_conv1d_validate_bwd": (ctypes.c_int, [ctypes.POINTER(S6ConvBwdArgs)]),
    "s6_causal_conv1d_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(S6ConvProblem)]),
    "s6_causal_conv1d_fwd": (ctypes.c_int, [ctypes.POINTER(S6ConvFwdArgs), ctypes.c_void_p]),
    "s6_causal_conv1d_bwd": (ctypes.c_int, [ctypes.POINTER(S6ConvBwdArgs), ctypes.c_void_p]),
    "s6_ssd_validate_fwd": (ctypes.c_int, [ctypes.POINTER(S6SsdFwdArgs)]),
    "s6_ssd_fwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(S6SsdProblem)]),
    "s6_ssd_fwd": (ctypes.c_int, [ctypes.POINTER(S6SsdFwdArgs), ctypes.c_void_p]),
    "s6_ssd_validate_bwd": (ctypes.c_int, [ctypes.POINTER(S6SsdBwdArgs)]),
    "s6_ssd_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(S6SsdProblem)]),
    "s6_ssd_bwd": (ctypes.c_int, [ctypes.POINTER(S6SsdBwdArgs), ctypes.c_void_p]),
    "s6_validate_state_update": (ctypes.c_int, [ctypes.POINTER(S6StateUpdateArgs)]),
    "s6_selective_state_update": (ctypes.c_int, [ctypes.POINTER(S6StateUpdateArgs), ctypes.c_void_p]),
}


def load_library(path=LIB_PATH):
    if not os.path.exists(path):
        raise ImportError(
            f"s6scan: native library not found at {path}; build it with "
            "`python ml-experiments_amd/build.py` (there is no non-HIP fallback)")
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:
        raise ImportError(f"s6scan: cannot load {path}: {e}") from e
    for name, (res, args) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.s6_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f"s6scan: library ABI version {ver}, expected {ABI_VERSION}")
    return lib


LIB = load_library()


def last_error():
    msg = LIB.s6_last_error()
    return msg.decode() if msg else ""


def check(rc, what):
    if rc != OK:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")
