"""ctypes binding of ``libmlpmk.so`` (declared in ``include/mlpmk.h``).

The library is loaded lazily on first use so that importing the package works
on machines without the built library; any call then raises ``OSError``
naming the missing file.  There is no fallback implementation.

``MLPMK_LIBRARY`` (environment) names another build of the same ABI to load
instead (a build with other compile-time options, for measurement).
"""
import ctypes
import os
import threading

LIB_NAME = "libmlpmk.so"
LIB_PATH = os.environ.get("MLPMK_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

c_int, c_int64, c_void_p, c_char_p = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_char_p
P_INT = ctypes.POINTER(c_int)
P_VOIDP = ctypes.POINTER(c_void_p)

# name -> (restype, argtypes); mirrors include/mlpmk.h
SIGNATURES = {
    "mlpmk_version": (c_int, []),
    "mlpmk_status_string": (c_char_p, [c_int]),
    "mlpmk_last_error": (c_char_p, []),
    "mlpmk_fwd_supported": (c_int, [c_int, P_INT]),
    "mlpmk_fwd_supported_dtype": (c_int, [c_int, P_INT, c_int]),
    "mlpmk_bwd_supported": (c_int, [c_int, P_INT]),
    "mlpmk_bwd_recompute_supported": (c_int, [c_int, P_INT]),
    "mlpmk_bwd_supported_dtype": (c_int, [c_int, P_INT, c_int]),
    "mlpmk_fwd": (c_int, [c_int, P_INT, c_int, c_void_p, P_VOIDP, c_void_p, P_VOIDP, c_int64, c_void_p]),
    "mlpmk_fwd_launch_info": (c_int, [c_int, P_INT, c_int, c_int64, c_int, P_INT]),
    "mlpmk_bwd": (
        c_int,
        [c_int, P_INT, c_int, c_void_p, P_VOIDP, P_VOIDP, c_void_p, c_int64, c_void_p, P_VOIDP, c_int64, c_void_p],
    ),
    "mlpmk_bwd_ws": (
        c_int,
        [c_int, P_INT, c_int, c_void_p, P_VOIDP, P_VOIDP, c_void_p, c_int64, c_void_p, P_VOIDP, c_void_p, c_int64,
         c_int64, c_void_p],
    ),
    "mlpmk_bwd_noalloc": (
        c_int,
        [c_int, P_INT, c_int, c_void_p, P_VOIDP, P_VOIDP, c_void_p, c_int64, c_void_p, P_VOIDP, c_int64, c_void_p],
    ),
    "mlpmk_bwd_workspace_size": (c_int, [c_int, P_INT, c_int, c_int64, c_int, ctypes.POINTER(c_int64)]),
    "mlpmk_wn_fwd": (c_int, [c_int, P_INT, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "mlpmk_wn_bwd": (
        c_int,
        [c_int, P_INT, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mlpmk_copy": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
    "mlpmk_sigmoid_h_mul": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int64, c_void_p]),
    "mlpmk_softplus_f32": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
}

STATUS = {
    0: "MLPMK_OK",
    1: "MLPMK_ERR_INVALID_ARG",
    2: "MLPMK_ERR_UNSUPPORTED_SHAPE",
    3: "MLPMK_ERR_MISALIGNED",
    4: "MLPMK_ERR_HIP",
    5: "MLPMK_ERR_NO_DEVICE",
}
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
BWD_WRITE_DW = 0x100  # MLPMK_BWD_WRITE_DW: OR-ed into the backward's dtype, dW written instead of accumulated

_lock = threading.Lock()
_lib = None


def get():
    """The loaded library (``ctypes.CDLL``) with argument types set."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise OSError(
                        f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                        "(hipcc --offload-arch=gfx950); there is no fallback path"
                    )
                lib = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(lib, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = lib
    return _lib


_int_arrays = {}


def int_array(vals):
    """A C int array of ``vals`` (cached per distinct tuple: the library only
    reads it).  Returns ``(array, keepalive)``; ctypes passes an array where
    the signature wants a pointer to its element type."""
    key = tuple(int(v) for v in vals)
    arr = _int_arrays.get(key)
    if arr is None:
        arr = (c_int * len(key))(*key)
        _int_arrays[key] = arr
    return arr, arr


def dims_array(key):
    """``int_array`` for a tuple of Python ints, returning the array alone
    (the launch paths' form: one dictionary lookup)."""
    arr = _int_arrays.get(key)
    if arr is None:
        arr = _int_arrays[key] = (c_int * len(key))(*key)
    return arr


def ptr_array(ptrs):
    """A C array of device pointers (None for NULL); ``(array, keepalive)``."""
    arr = (c_void_p * len(ptrs))(*ptrs)
    return arr, arr
