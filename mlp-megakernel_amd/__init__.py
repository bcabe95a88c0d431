"""MI355X (gfx950) fused softplus-MLP megakernel library.

Host side of ``libmlpmk.so``: ctypes bindings (``_lib``), torch-facing launch
wrappers (``ops``) and the autograd functions / modules (``autograd``).  The
HIP library is required: every entry point raises if it is missing.
"""
from . import _lib  # noqa: F401
from .ops import (  # noqa: F401
    MlpmkError,
    fwd,
    fwd_into,
    bwd,
    wn_fwd,
    wn_bwd,
    copy_bytes,
    fwd_supported,
    bwd_supported,
    library_path,
)

__all__ = [
    "MlpmkError",
    "fwd",
    "fwd_into",
    "bwd",
    "wn_fwd",
    "wn_bwd",
    "copy_bytes",
    "fwd_supported",
    "bwd_supported",
    "library_path",
]
