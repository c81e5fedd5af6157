"""s6scan: MI355X-native (gfx950 HIP) S6 selective scan behind the reference's
``selective_scan_fn`` / ``SelectiveScanFn`` interface."""
from . import _lib  # noqa: F401  (loads libs6scan.so; ImportError if it is missing)
from .selective_scan_interface import (  # noqa: F401
    SelectiveScanFn,
    check_inputs,
    selective_scan_backward,
    selective_scan_fn,
    selective_scan_forward,
)

__all__ = ["SelectiveScanFn", "selective_scan_fn", "selective_scan_forward",
           "selective_scan_backward", "check_inputs"]
