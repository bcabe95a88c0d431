"""Torch-facing launch wrappers over the C ABI of ``libmlpmk.so``.

Tensors only supply device pointers and the stream: every launch goes through
``include/mlpmk.h`` on the caller's current torch stream of the tensor's
device.  Validation errors of the library surface as ``MlpmkError``.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


class MlpmkError(RuntimeError):
    """A non-zero ``mlpmk_status`` returned by the library."""

    def __init__(self, fn, status, detail):
        self.status = status
        name = _lib.STATUS.get(status, f"status {status}")
        super().__init__(f"{fn} failed: {name}: {detail}")


def library_path():
    return _lib.LIB_PATH


def _check(fn, rc):
    if rc != 0:
        lib = _lib.get()
        detail = lib.mlpmk_last_error().decode(errors="replace")
        raise MlpmkError(fn, rc, detail)


def _dims_of(x, weights):
    dims = [int(x.shape[1])] + [int(w.shape[1]) for w in weights]
    for i, w in enumerate(weights):
        if w.dim() != 2 or int(w.shape[0]) != dims[i]:
            raise ValueError(
                f"weight {i} has shape {tuple(w.shape)}; expected [{dims[i]}, out] chained on x {tuple(x.shape)}"
            )
    return dims


def fwd_supported(dims, dtype=None):
    """True if a fused forward kernel takes ``dims`` (for tensors of
    ``dtype``; default: any element type, ``mlpmk_fwd_supported``)."""
    lib = _lib.get()
    p, _keep = _lib.int_array(dims)
    if dtype is None:
        return bool(lib.mlpmk_fwd_supported(len(dims) - 1, p))
    return bool(lib.mlpmk_fwd_supported_dtype(len(dims) - 1, p, _fwd_code(dtype)))


def bwd_supported(dims, dtype=None):
    """True if a backward kernel takes ``dims`` (for tensors of ``dtype``;
    default: 16-bit tensors, ``mlpmk_bwd_supported``)."""
    lib = _lib.get()
    p, _keep = _lib.int_array(dims)
    if dtype is None:
        return bool(lib.mlpmk_bwd_supported(len(dims) - 1, p))
    return bool(lib.mlpmk_bwd_supported_dtype(len(dims) - 1, p, _fwd_code(dtype)))


def bwd_recompute_supported(dims):
    """True if the backward recomputes h_{L-1} when its stash entry is None
    (``mlpmk_bwd_recompute_supported``; no dx in that mode)."""
    lib = _lib.get()
    p, _keep = _lib.int_array(dims)
    return bool(lib.mlpmk_bwd_recompute_supported(len(dims) - 1, p))


# Element types of the megakernels' 16-bit tensors (x, weights, out, dout, dx).
_ELEM = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}


def _elem_code(dtype, name="x"):
    code = _ELEM.get(dtype)
    if code is None:
        raise TypeError(f"{name} must be float16 or bfloat16, got {dtype} (cast first: fp32 accumulation either way)")
    return code


def _fwd_code(dtype, name="x"):
    """Element type of x, weights, out (and dout, dx): fp16, bf16, or fp32
    (fp32 tensors run with bf16 hi/lo split MFMA operands and fp32 rows)."""
    if dtype == torch.float32:
        return _lib.DTYPE_F32
    code = _ELEM.get(dtype)
    if code is None:
        raise TypeError(f"{name} must be float32, float16 or bfloat16, got {dtype}")
    return code


def _ok(t, dtype, device):
    """The checks of ``_require`` as one boolean (no name formatting on the
    launch path; ``_require`` then names what failed)."""
    return isinstance(t, torch.Tensor) and t.dtype == dtype and t.device == device and t.is_contiguous()


def _require(t, name, dtype, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
# Current device without torch.cuda.current_device()'s Python layers (~1 us).
_cur_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _stream_of(dev):
    """The raw current stream of ``dev`` when ``dev`` is the current device
    (or names none), else None: the caller switches first.  The raw queries
    cost ~0.1 us against ~3 us for ``current_stream().cuda_stream``."""
    cur = _cur_device()
    if dev.index is not None and dev.index != cur:
        return None
    return _raw_stream(cur) if _raw_stream is not None else torch.cuda.current_stream(cur).cuda_stream


def _launch(dev, fn, *args):
    """``fn(*args, stream)`` with ``dev`` current: the library launches on the
    calling thread's current HIP device.  Switches only when needed (the
    device context manager costs ~2.4 us per call)."""
    st = _stream_of(dev)
    if st is not None:
        return fn(*args, st)
    with torch.cuda.device(dev.index):
        return fn(*args, _stream_of(dev))


# Pointer-level launches.  The public wrappers below validate tensors and call
# these; the autograd Functions call them directly for buffers they allocated
# themselves (shapes known), which keeps a training step's host time down.
# ``dims`` is a tuple of ints; pointers are ints (None for NULL).  They go
# through the CPython shims of ``_mlpmk_launch`` (csrc/pylaunch.c, bound to
# the entry points of the library ctypes loaded) when that module is built,
# else through ctypes.
try:
    from . import _mlpmk_launch as _shim
except ImportError:  # not built: ctypes only
    _shim = None
_shim_lib = None  # the ctypes library whose entry points the shim is bound to


def _fast():
    """The shim module bound to the current library, or None."""
    global _shim_lib
    lib = _lib.get()
    if _shim is None:
        return None
    if _shim_lib is not lib:
        addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value  # noqa: E731
        _shim.bind(addr(lib.mlpmk_fwd), addr(lib.mlpmk_bwd), addr(lib.mlpmk_bwd_ws), addr(lib.mlpmk_wn_fwd),
                   addr(lib.mlpmk_wn_bwd))
        _shim_lib = lib
    return _shim


def _fwd_raw(dev, dims, code, x_ptr, w_ptrs, out_ptr, stash_ptrs, M):
    f = _fast()
    if f is not None:
        rc = _launch(dev, f.fwd, dims, code, x_ptr, w_ptrs, out_ptr, stash_ptrs, M)
    else:
        lib = _lib.get()
        L = len(dims) - 1
        pw = (_lib.c_void_p * L)(*w_ptrs)
        ps = None if stash_ptrs is None else (_lib.c_void_p * (L - 1))(*stash_ptrs)
        rc = _launch(dev, lib.mlpmk_fwd, L, _lib.dims_array(dims), code, x_ptr, pw, out_ptr, ps, M)
    if rc:
        _check("mlpmk_fwd", rc)


def _bwd_raw(dev, dims, code, x_ptr, w_ptrs, stash_ptrs, dout_ptr, row_stride, dx_ptr, dw_ptrs, M, workspace=True):
    ws, nbytes = None, 0
    if workspace and M > 0:
        nbytes = _workspace_bytes(dev.index if dev.index is not None else _cur_device(), dims, M, dx_ptr is not None,
                                  code)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    name = "mlpmk_bwd_ws" if ws is not None else "mlpmk_bwd"
    f = _fast()
    if f is not None:
        rc = _launch(dev, f.bwd, dims, code, x_ptr, w_ptrs, stash_ptrs, dout_ptr, row_stride, dx_ptr, dw_ptrs,
                          ws.data_ptr() if ws is not None else None, nbytes, M)
    else:
        lib = _lib.get()
        L = len(dims) - 1
        pd = _lib.dims_array(dims)
        pw = (_lib.c_void_p * L)(*w_ptrs)
        ps = (_lib.c_void_p * (L - 1))(*stash_ptrs)
        pg = (_lib.c_void_p * L)(*dw_ptrs)
        if ws is not None:
            rc = _launch(dev, lib.mlpmk_bwd_ws, L, pd, code, x_ptr, pw, ps, dout_ptr, row_stride, dx_ptr, pg,
                         ws.data_ptr(), nbytes, M)
        else:
            rc = _launch(dev, lib.mlpmk_bwd, L, pd, code, x_ptr, pw, ps, dout_ptr, row_stride, dx_ptr, pg, M)
    if rc:
        _check(name, rc)


def _wn_fwd_raw(dev, dims, pcode, wcode, v_ptr, g_ptr, w_ptr, inv_ptr):
    f = _fast()
    if f is not None:
        rc = _launch(dev, f.wn_fwd, dims, pcode, wcode, v_ptr, g_ptr, w_ptr, inv_ptr)
    else:
        rc = _launch(dev, _lib.get().mlpmk_wn_fwd, len(dims) - 1, _lib.dims_array(dims), pcode, wcode, v_ptr, g_ptr,
                     w_ptr, inv_ptr)
    if rc:
        _check("mlpmk_wn_fwd", rc)


def _wn_bwd_raw(dev, dims, pcode, dw_ptr, v_ptr, g_ptr, inv_ptr, dv_ptr, dg_ptr):
    f = _fast()
    if f is not None:
        rc = _launch(dev, f.wn_bwd, dims, pcode, dw_ptr, v_ptr, g_ptr, inv_ptr, dv_ptr, dg_ptr)
    else:
        rc = _launch(dev, _lib.get().mlpmk_wn_bwd, len(dims) - 1, _lib.dims_array(dims), pcode, dw_ptr, v_ptr, g_ptr,
                     inv_ptr, dv_ptr, dg_ptr)
    if rc:
        _check("mlpmk_wn_bwd", rc)


DOUT_SCALAR = -1  # MLPMK_DOUT_SCALAR


def _dout_rows(dout, M, out_w, dtype, dev):
    """``(dout, row_stride)`` as the library reads it: one element broadcast
    everywhere (both strides 0: ``DOUT_SCALAR``), or [M, OUT] rows with unit
    column stride whose row stride (0 for a broadcast row) is a multiple of 8
    elements and whose first element is 16-byte aligned; other row strides
    and base addresses (a column slice of a wider gradient) are copied into
    padded rows."""
    if dout.dtype != dtype or dout.device != dev:
        raise TypeError(f"dout must be {dtype} on the same device as x")
    if tuple(dout.shape) != (M, out_w):
        raise ValueError(f"dout must be [M, OUT]={M, out_w}")
    if dout.stride() == (0, 0):  # (M = 0 too: the library then reads nothing)
        return dout, DOUT_SCALAR
    if dout.stride(1) != 1:
        raise ValueError(f"dout must be [M, OUT]={M, out_w} with unit column stride")
    row_stride = int(dout.stride(0)) if M > 1 else -(-out_w // 8) * 8
    if row_stride % 8 != 0 or dout.data_ptr() % 16 != 0:
        # The library reads dout rows from 16-byte boundaries: an output width
        # that is not a multiple of 8, or rows that start off such a boundary,
        # get a padded copy.
        padded = torch.zeros((M, -(-out_w // 8) * 8), dtype=dtype, device=dev)
        padded[:, :out_w] = dout
        dout, row_stride = padded, padded.shape[1]
    return dout, row_stride


def fwd_into(x, weights, out, stash=None):
    """Run the forward megakernel writing ``out`` (and ``stash`` if given).

    ``x`` [M, D] fp16, bf16 or fp32, ``weights`` list of [in, out] and
    ``out`` [M, OUT] of x's dtype, ``stash`` list of L-1 fp32 [M, H_l] tensors
    (an entry may be None: that activation is not written) or None.  All
    contiguous on one CUDA (HIP) device.  fp32 tensors run with bf16 hi/lo
    split MFMA operands (fp32's exponent range, a ~16-bit significand) and
    fp32 accumulation, softplus and output rows.
    """
    dev = x.device
    if dev.type != "cuda":
        raise ValueError(f"x must be on a GPU device, got {dev}")
    xd = x.dtype
    code = _fwd_code(xd)
    if not x.is_contiguous():
        _require(x, "x", xd, dev)
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [M, D], got shape {tuple(x.shape)}")
    for i, w in enumerate(weights):
        if not _ok(w, xd, dev):
            _require(w, f"w{i + 1}", xd, dev)
    dims = _dims_of(x, weights)
    M = int(x.shape[0])
    if not _ok(out, xd, dev):
        _require(out, "out", xd, dev)
    if tuple(out.shape) != (M, dims[-1]):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {(M, dims[-1])}")
    stash_ptrs = None
    if stash is not None:
        if len(stash) != len(weights) - 1:
            raise ValueError(f"stash needs {len(weights) - 1} tensors, got {len(stash)}")
        for i, s in enumerate(stash):
            if s is None:
                continue
            if not _ok(s, torch.float32, dev):
                _require(s, f"stash[{i}]", torch.float32, dev)
            if tuple(s.shape) != (M, dims[i + 1]):
                raise ValueError(f"stash[{i}] has shape {tuple(s.shape)}, expected {(M, dims[i + 1])}")
        stash_ptrs = [s.data_ptr() if s is not None else None for s in stash]
    _fwd_raw(dev, tuple(dims), code, x.data_ptr(), [w.data_ptr() for w in weights], out.data_ptr(), stash_ptrs, M)
    return out


KERNEL_NAMES = {-1: "none", 0: "persistent", 1: "feature_split"}


def fwd_launch_info(dims, M, stash=False, dtype=torch.float16, device=None):
    """The launch ``mlpmk_fwd`` makes for this shape on ``device`` (default:
    the current one), from the library's own dispatch code, without
    launching: ``{"kernel", "rows_per_block", "waves", "grid", "wgs_per_cu"}``
    (``mlpmk_fwd_launch_info``)."""
    lib = _lib.get()
    pd, _k = _lib.int_array(list(dims))
    info = (ctypes.c_int * 5)()
    idx = torch.cuda.current_device() if device is None or device.index is None else device.index
    with torch.cuda.device(idx):
        rc = lib.mlpmk_fwd_launch_info(len(dims) - 1, pd, _fwd_code(dtype), int(M), int(bool(stash)), info)
    _check("mlpmk_fwd_launch_info", rc)
    return {"kernel": KERNEL_NAMES[info[0]], "rows_per_block": info[1], "waves": info[2], "grid": info[3],
            "wgs_per_cu": info[4]}


def fwd(x, weights, stash=False, recompute=False):
    """Allocate ``out`` (and the fp32 stash when ``stash``) and run the forward.

    Returns ``out`` or ``(out, [h1, ..., h_{L-1}])``.  With ``recompute`` the
    last entry is None and h_{L-1} is not written: the backward recomputes it
    (``bwd_recompute_supported``).
    """
    dims = _dims_of(x, weights)
    M = int(x.shape[0])
    out = torch.empty((M, dims[-1]), device=x.device, dtype=x.dtype)
    hs = None
    if stash:
        hs = [torch.empty((M, d), device=x.device, dtype=torch.float32) for d in dims[1:-1]]
        if recompute:
            if not bwd_recompute_supported(dims):
                raise ValueError(f"no recomputing backward for widths {dims}: stash every activation")
            hs[-1] = None
    fwd_into(x, weights, out, hs)
    return (out, hs) if stash else out


_ws_bytes = {}


def bwd_workspace_bytes(dims, M, with_dx, device=None, dtype=torch.float16):
    """Bytes of workspace ``mlpmk_bwd_ws`` needs on ``device`` (default: the
    current device) for tensors of ``dtype``; cached per device, shape and M."""
    idx = _cur_device() if device is None or device.index is None else device.index
    return _workspace_bytes(idx, tuple(int(d) for d in dims), int(M), bool(with_dx), _fwd_code(dtype))


def _workspace_bytes(idx, dims, M, with_dx, code):
    key = (idx, dims, M, with_dx, code)
    n = _ws_bytes.get(key)
    if n is None:
        lib = _lib.get()
        out = ctypes.c_int64(0)
        with torch.cuda.device(idx):
            rc = lib.mlpmk_bwd_workspace_size(len(dims) - 1, _lib.dims_array(dims), code, M, int(with_dx),
                                              ctypes.byref(out))
        _check("mlpmk_bwd_workspace_size", rc)
        n = _ws_bytes[key] = out.value
    return n


def bwd(x, weights, stash, dout, dws, dx=None, workspace=True, accumulate=True):
    """Backward megakernel: accumulates fp32 weight gradients into ``dws``
    (callers zero them first), or with ``accumulate=False`` writes them
    (``MLPMK_BWD_WRITE_DW``: their prior contents do not matter), and
    writes ``dx`` if given.

    ``x``, the weights, ``dout`` and ``dx`` are fp16, bf16 or fp32 (fp32
    tensors run with bf16 hi/lo split operands: fp32's exponent range).
    ``dout`` is [M, OUT] of x's dtype with unit column stride; a row stride of 0
    (``t.expand(M, OUT)`` of one row) is passed through as a broadcast, and
    so is one element expanded over both dimensions (what ``loss =
    out.sum()`` hands back: ``MLPMK_DOUT_SCALAR``, no copy).
    With ``workspace`` (default) the weight-gradient partials of the
    workgroups go through a workspace from torch's allocator and a second
    kernel (``mlpmk_bwd_ws``); otherwise every workgroup adds its partials
    with fp32 atomics (``mlpmk_bwd``).  A None last stash entry selects the
    recomputing backward (``bwd_recompute_supported``; with or without dx).
    """
    dev = x.device
    xd = x.dtype
    code = _fwd_code(xd) | (0 if accumulate else _lib.BWD_WRITE_DW)
    if not _ok(x, xd, dev):
        _require(x, "x", xd, dev)
    for i, w in enumerate(weights):
        if not _ok(w, xd, dev):
            _require(w, f"w{i + 1}", xd, dev)
    dims = _dims_of(x, weights)
    M = int(x.shape[0])
    if len(stash) != len(weights) - 1:
        raise ValueError(f"stash needs {len(weights) - 1} tensors, got {len(stash)}")
    for i, s in enumerate(stash):
        if s is None and i == len(stash) - 1:
            continue  # recompute mode: the library checks that the shape has it
        if not _ok(s, torch.float32, dev):
            _require(s, f"stash[{i}]", torch.float32, dev)
        if tuple(s.shape) != (M, dims[i + 1]):
            raise ValueError(f"stash[{i}] has shape {tuple(s.shape)}, expected {(M, dims[i + 1])}")
    for i, d in enumerate(dws):
        if not _ok(d, torch.float32, dev):
            _require(d, f"dw[{i}]", torch.float32, dev)
        if tuple(d.shape) != (dims[i], dims[i + 1]):
            raise ValueError(f"dw[{i}] has shape {tuple(d.shape)}, expected {(dims[i], dims[i + 1])}")
    dout, row_stride = _dout_rows(dout, M, dims[-1], x.dtype, dev)
    if dx is not None:
        _require(dx, "dx", x.dtype, dev)
        if tuple(dx.shape) != (M, dims[0]):
            raise ValueError(f"dx has shape {tuple(dx.shape)}, expected {(M, dims[0])}")
    _bwd_raw(dev, tuple(dims), code, x.data_ptr(), [w.data_ptr() for w in weights],
             [s.data_ptr() if s is not None else None for s in stash], dout.data_ptr(), row_stride,
             dx.data_ptr() if dx is not None else None, [d.data_ptr() for d in dws], M, workspace)
    return dws, dx


def _param_dtype(t):
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    if t.dtype == torch.float16:
        return _lib.DTYPE_F16
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    raise TypeError(f"weight-norm parameters must be fp32, fp16 or bf16, got {t.dtype}")


def wn_fwd(dims, v_all, g_all, w_all, inv_all):
    """``W = g v / ||v||`` for all layers in one launch (flat contiguous blocks)."""
    dev = v_all.device
    dt = _param_dtype(v_all)
    _require(v_all, "v_all", v_all.dtype, dev)
    _require(g_all, "g_all", v_all.dtype, dev)
    wcode = _fwd_code(w_all.dtype, "w_all")
    _require(w_all, "w_all", w_all.dtype, dev)
    _require(inv_all, "inv_all", torch.float32, dev)
    nw = sum(dims[i] * dims[i + 1] for i in range(len(dims) - 1))
    ng = sum(dims[1:])
    if v_all.numel() != nw or w_all.numel() != nw or g_all.numel() != ng or inv_all.numel() != ng:
        raise ValueError("weight-norm block sizes do not match dims")
    _wn_fwd_raw(dev, tuple(int(d) for d in dims), dt, wcode, v_all.data_ptr(), g_all.data_ptr(), w_all.data_ptr(),
                inv_all.data_ptr())
    return w_all, inv_all


def wn_bwd(dims, dw_all, v_all, g_all, inv_all, dv_all, dg_all):
    """``dW -> (dv, dg)`` for all layers in one launch."""
    dev = v_all.device
    dt = _param_dtype(v_all)
    _require(dw_all, "dw_all", torch.float32, dev)
    _require(v_all, "v_all", v_all.dtype, dev)
    _require(g_all, "g_all", v_all.dtype, dev)
    _require(inv_all, "inv_all", torch.float32, dev)
    _require(dv_all, "dv_all", v_all.dtype, dev)
    _require(dg_all, "dg_all", v_all.dtype, dev)
    nw = sum(dims[i] * dims[i + 1] for i in range(len(dims) - 1))
    ng = sum(dims[1:])
    if dw_all.numel() != nw or v_all.numel() != nw or dv_all.numel() != nw:
        raise ValueError("weight-norm block sizes do not match dims")
    if g_all.numel() != ng or inv_all.numel() != ng or dg_all.numel() != ng:
        raise ValueError("weight-norm block sizes do not match dims")
    _wn_bwd_raw(dev, tuple(int(d) for d in dims), dt, dw_all.data_ptr(), v_all.data_ptr(), g_all.data_ptr(),
                inv_all.data_ptr(), dv_all.data_ptr(), dg_all.data_ptr())
    return dv_all, dg_all


def copy_bytes(src, dst):
    """Calibration copy of ``src`` into ``dst`` (same byte size, multiple of 16)."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("copy size mismatch")
    lib = _lib.get()
    rc = _launch(src.device, lib.mlpmk_copy, src.data_ptr(), dst.data_ptr(), nbytes)
    _check("mlpmk_copy", rc)
    return dst
