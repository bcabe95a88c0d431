"""The C ABI of libmlpmk.so on the CPU: it loads, exports every symbol that
include/mlpmk.h declares, and its host-side validation rejects bad arguments
with the documented status codes before anything touches a device.  No
compute is launched here (this container has no GPU)."""
import ctypes
import os
import re

import pytest
import torch

import mlpmk
from mlpmk import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mlpmk.h")

OK, INVALID, UNSUPPORTED, MISALIGNED, HIPERR, NODEV = 0, 1, 2, 3, 4, 5
A = 0x10000  # a fake, 16-byte aligned device address (never dereferenced)


def declared_symbols():
    text = open(HEADER).read()
    # function declarations: a return type at the start of a line, then the name
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(mlpmk_[a-z0-9_]+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol():
    lib = _lib.get()
    names = declared_symbols()
    assert "mlpmk_fwd" in names and "mlpmk_bwd" in names and "mlpmk_wn_fwd" in names
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"


def test_version_and_status_strings():
    lib = _lib.get()
    assert lib.mlpmk_version() >= 204  # MLPMK_DOUT_SCALAR (201), MLPMK_BWD_WRITE_DW (203), mlpmk_softplus_f32 (204)
    for code, text in [(0, b"ok"), (2, b"unsupported shape"), (5, b"no usable gfx950 device")]:
        assert lib.mlpmk_status_string(code) == text
    assert lib.mlpmk_status_string(99) == b"unknown status"


@pytest.mark.parametrize(
    "dims,ok,bwd_ok",
    [((128, 128, 128, 128), True, True), ((128,) * 6, True, True), ((32, 64, 64, 16), True, True),
     # runtime-width kernels: 2..5 layers, input/hidden multiples of 16 up to
     # 128, any output width up to 128
     ((128, 64, 128, 128), True, True), ((32, 128, 3), True, True), ((16, 48, 80, 112, 7), True, True),
     ((128,) * 5, True, True), ((64, 128, 128, 1), True, True),
     # streamed-weight forward: widths up to 256 (multiples of 16, any output
     # width up to 256); the two-pass backward takes them when the output
     # width is a multiple of 8 (else the modules train through the
     # library-GEMM fallback)
     ((128, 256, 128), True, True), ((128, 256, 256, 128), True, True), ((256, 64, 200), True, True),
     ((128, 128, 129), True, False), ((16, 256, 256, 256, 256, 256), True, True), ((128, 256, 132), True, False),
     ((128, 128), False, False), ((100, 128, 128, 128), False, False), ((128, 136, 128, 128), False, False),
     ((128, 272, 128), False, False), ((128, 128, 257), False, False), ((128, 248, 128), False, False),
     ((128,) * 7, False, False)],
)
def test_forward_support_table(dims, ok, bwd_ok):
    assert ops.fwd_supported(list(dims)) is ok
    assert ops.bwd_supported(list(dims)) is bwd_ok


def _fwd(dims, x=A, w=(A, A, A), out=A, stash=None, m=256, dtype=1):
    lib = _lib.get()
    pd, _k1 = _lib.int_array(dims)
    pw, _k2 = _lib.ptr_array(list(w))
    ps, _k3 = (_lib.ptr_array(list(stash)) if stash is not None else (None, None))
    return lib.mlpmk_fwd(len(dims) - 1, pd, dtype, x, pw, out, ps, m, None)


def test_fwd_validation_codes():
    lib = _lib.get()
    d = [128, 128, 128, 128]
    assert _fwd(d, m=-1) == INVALID
    assert _fwd([128, 100, 128, 128]) == UNSUPPORTED
    assert _fwd([128, 128]) == UNSUPPORTED  # one layer
    assert _fwd(d, x=A + 2) == MISALIGNED
    assert _fwd(d, out=None) == INVALID
    assert _fwd(d, w=(A, A + 8, A)) == MISALIGNED
    assert _fwd(d, stash=(A, A + 4)) == MISALIGNED
    assert b"stash[1]" in lib.mlpmk_last_error()
    assert lib.mlpmk_fwd(3, None, 1, A, None, A, None, 1, None) == INVALID
    # element types: fp16 (1), bf16 (2) and fp32 (0, bf16 hi/lo split operands); others are invalid
    assert _fwd(d, dtype=7) == INVALID
    assert _fwd(d, dtype=0, m=0) == OK
    assert _fwd(d, dtype=2, m=0) == OK
    # M == 0 succeeds without touching a device (x/out may even be NULL)
    assert _fwd(d, x=None, out=None, m=0) == OK
    # valid arguments reach the device query, which fails without a GPU; a
    # NULL stash entry is valid (that activation is not written)
    if not torch.cuda.is_available():
        assert _fwd(d) in (NODEV, HIPERR)
        assert lib.mlpmk_last_error() != b""
        assert _fwd(d, stash=(A, None)) in (NODEV, HIPERR)
        assert _fwd(d, dtype=2) in (NODEV, HIPERR)
        assert _fwd(d, dtype=0) in (NODEV, HIPERR)


def test_bwd_validation_codes():
    lib = _lib.get()
    d = [128, 128, 128, 128]
    pd, _k1 = _lib.int_array(d)
    pw, _k2 = _lib.ptr_array([A, A, A])
    ps, _k3 = _lib.ptr_array([A, A])
    pg, _k4 = _lib.ptr_array([A, A, A])
    call = lambda **kw: lib.mlpmk_bwd(  # noqa: E731
        3, pd, kw.get("dtype", 1), kw.get("x", A), pw, kw.get("stash", ps), kw.get("dout", A), kw.get("stride", 128),
        kw.get("dx", None), kw.get("dw", pg), kw.get("m", 256), None)
    assert call(m=-1) == INVALID
    assert call(stride=-2) == INVALID  # negative, and not MLPMK_DOUT_SCALAR
    assert call(dw=None) == INVALID
    # fp32 tensors run the two-pass backward, which hands dz between its
    # passes through the workspace: mlpmk_bwd (none) refuses them
    assert call(dtype=0) == INVALID and b"mlpmk_bwd_ws" in lib.mlpmk_last_error()
    assert call(dtype=3) == INVALID
    # MLPMK_BWD_WRITE_DW (0x100) rides in the dtype argument: validated like the
    # bare type, an unknown type with it is still invalid
    assert call(dtype=1 | 0x100, m=-1) == INVALID and call(dtype=3 | 0x100) == INVALID
    assert call(dtype=0 | 0x100) == INVALID and b"mlpmk_bwd_ws" in lib.mlpmk_last_error()
    if not torch.cuda.is_available() and ops.bwd_supported(d):
        # an empty batch with dW written still writes dW = 0: a launch, which needs the device
        assert call(dtype=1 | 0x100, m=0) in (NODEV, HIPERR)
    if ops.bwd_supported(d):
        assert call(stride=64) == INVALID  # below the output width
        assert call(stride=130) == MISALIGNED
        assert call(dout=A + 4) == MISALIGNED
        assert call(m=0) == OK
        # MLPMK_DOUT_SCALAR: one element, 2-byte aligned, any output width
        assert call(stride=-1, dout=A + 1) == MISALIGNED
        assert call(stride=-1, dout=A + 2, m=0) == OK
    else:
        assert call() == UNSUPPORTED


@pytest.mark.parametrize("dims,ok", [((128, 128, 128, 128), True), ((128,) * 6, True), ((32, 64, 64, 16), False),
                                     ((128, 128, 128), False), ((128, 64, 128, 128), False), ((128,) * 5, False),
                                     ((128, 256, 256, 128), False)])
def test_recompute_support_table(dims, ok):
    assert ops.bwd_recompute_supported(list(dims)) is ok


def test_recompute_needs_a_supported_shape_in_the_python_layer():
    x = torch.zeros((4, 32), dtype=torch.float16)
    ws = [torch.zeros((32, 64), dtype=torch.float16), torch.zeros((64, 64), dtype=torch.float16),
          torch.zeros((64, 16), dtype=torch.float16)]
    with pytest.raises(ValueError, match="recomputing"):
        ops.fwd(x, ws, stash=True, recompute=True)


def test_recompute_validation_codes():
    # stash[L-2] == NULL selects the recomputing backward where it exists
    # (with or without dx); every other NULL stash entry is rejected on the host.
    lib = _lib.get()
    pw, _k2 = _lib.ptr_array([A, A, A])
    pg, _k4 = _lib.ptr_array([A, A, A])
    pd, _k1 = _lib.int_array([128] * 4)

    def call(stash, dx=None, dims=pd, n=3, w=pw, g=pg):
        ps, _k = _lib.ptr_array(list(stash))
        return lib.mlpmk_bwd(n, dims, 1, A, w, ps, A, 128, dx, g, 256, None)

    assert call((None, A)) == INVALID
    assert b"stash[0]" in lib.mlpmk_last_error()
    pn, _k5 = _lib.int_array([32, 64, 64, 16])
    assert call((A, None), dims=pn) == INVALID  # no recomputing kernel for this shape
    if not torch.cuda.is_available():
        assert call((A, None)) in (NODEV, HIPERR)  # valid: reaches the device query
        assert call((A, None), dx=A) in (NODEV, HIPERR)


def test_5l_backward_is_supported_but_needs_a_workspace():
    lib = _lib.get()
    d = [128] * 6
    pd, _k1 = _lib.int_array(d)
    assert ops.bwd_supported(d)
    pw, _k2 = _lib.ptr_array([A] * 5)
    ps, _k3 = _lib.ptr_array([A] * 4)
    pg, _k4 = _lib.ptr_array([A] * 5)
    # Rejected before any device call: dz travels between two launches through the workspace.
    assert lib.mlpmk_bwd(5, pd, 1, A, pw, ps, A, 128, None, pg, 256, None) == INVALID
    assert b"mlpmk_bwd_ws" in lib.mlpmk_last_error()


def test_wn_and_copy_validation_codes():
    lib = _lib.get()
    pd, _k = _lib.int_array([128, 128, 128, 128])
    assert lib.mlpmk_wn_fwd(3, pd, 7, 1, A, A, A, A, None) == INVALID  # bad dtype
    assert lib.mlpmk_wn_fwd(3, pd, 0, 3, A, A, A, A, None) == INVALID  # W is fp32, fp16 or bf16
    assert b"w_dtype" in lib.mlpmk_last_error()
    assert lib.mlpmk_wn_fwd(3, pd, 0, 1, A, None, A, A, None) == INVALID
    assert lib.mlpmk_wn_bwd(3, pd, 1, A, A, A, A, A + 2, A, None) == MISALIGNED
    pbad, _k2 = _lib.int_array([128, 0, 128, 128])
    assert lib.mlpmk_wn_fwd(3, pbad, 0, 1, A, A, A, A, None) == INVALID  # any positive widths
    assert lib.mlpmk_copy(A, A, 17, None) == INVALID
    assert lib.mlpmk_copy(A, A, 0, None) == OK


def test_elementwise_validation_codes():
    lib = _lib.get()
    assert lib.mlpmk_softplus_f32(A, A, -1, None) == INVALID
    assert lib.mlpmk_softplus_f32(A, A, 0, None) == OK
    assert lib.mlpmk_softplus_f32(None, A, 4, None) == INVALID
    assert lib.mlpmk_softplus_f32(A, A + 4, 4, None) == MISALIGNED
    assert b"h=" in lib.mlpmk_last_error()
    assert lib.mlpmk_sigmoid_h_mul(A, A, 7, A, None, 1, 4, None) == INVALID  # dh fp32, fp16 or bf16
    assert lib.mlpmk_sigmoid_h_mul(A, A, 1, A, A, 0, 4, None) == INVALID  # dz16 is a 16-bit copy
    assert lib.mlpmk_sigmoid_h_mul(A, A, 1, A, None, 1, -1, None) == INVALID
    assert lib.mlpmk_sigmoid_h_mul(A, A, 1, A, None, 1, 0, None) == OK
    assert lib.mlpmk_sigmoid_h_mul(A, A + 2, 1, A, None, 1, 4, None) == MISALIGNED


@pytest.mark.parametrize("dims,f16,f32", [((128, 128, 128, 128), 1, 1), ((64, 96, 3), 1, 1),
                                          ((128, 256, 128), 1, 0), ((128, 320, 128), 0, 0),
                                          ((3, 64, 64), 0, 0), ((16,) * 7, 0, 0)])
def test_forward_support_by_dtype(dims, f16, f32):
    # fp32 tensors have fused kernels up to width 128; 16-bit ones up to 256.
    lib = _lib.get()
    p, _k = _lib.int_array(list(dims))
    L = len(dims) - 1
    assert lib.mlpmk_fwd_supported_dtype(L, p, _lib.DTYPE_F16) == f16
    assert lib.mlpmk_fwd_supported_dtype(L, p, _lib.DTYPE_BF16) == f16
    assert lib.mlpmk_fwd_supported_dtype(L, p, _lib.DTYPE_F32) == f32
    assert lib.mlpmk_fwd_supported_dtype(L, p, 7) == 0
    assert ops.fwd_supported(list(dims), torch.float32) is bool(f32)


def test_python_wrappers_validate_before_the_library():
    x = torch.zeros((4, 128), dtype=torch.float16)
    ws = [torch.zeros((128, 128), dtype=torch.float16) for _ in range(3)]
    out = torch.empty((4, 128), dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        ops.fwd_into(x, ws, out)
    with pytest.raises(ValueError, match="weight 1"):
        ops._dims_of(x, [ws[0], torch.zeros((64, 128), dtype=torch.float16), ws[2]])


def test_drop_in_modules_import_without_gpu():
    import kernel

    # MI355X (256 CUs): feature-split kernel up to one 32-row block per CU
    # (two for the narrow network), then 4-, 8- and 12/16-wave workgroups.
    cfg = kernel._pick_config
    assert cfg(4096, 128, 128, 128, 128) == (32, 128, 16, 16, 16, 4)
    assert cfg(8192, 128, 128, 128, 128) == (32, 128, 16, 16, 16, 4)
    assert cfg(16384, 128, 128, 128, 128) == (32, 128, 16, 16, 16, 4)
    assert cfg(65536, 128, 128, 128, 128) == (32, 128, 16, 16, 16, 8)
    assert cfg(1048576, 128, 128, 128, 128) == (32, 128, 16, 16, 16, 12)
    assert cfg(4096, 32, 64, 64, 16) == (32, 16, 16, 16, 16, 2)
    assert cfg(16384, 32, 64, 64, 16) == (32, 16, 16, 16, 16, 2)
    assert cfg(40000, 32, 64, 64, 16) == (64, 16, 16, 16, 16, 4)
    assert cfg(4194304, 32, 64, 64, 16) == (64, 16, 16, 16, 16, 16)
    assert cfg(4096, 128, 128, 128, 128, num_cus=8) == (32, 128, 16, 16, 16, 12)
    # fp32 tensors: their layer pipeline at every M (32-row blocks, 4 waves per
    # layer of the 3-layer network)
    assert cfg(4096, 128, 128, 128, 128, fp32=True) == (32, 128, 16, 16, 16, 12)
    assert cfg(1048576, 128, 128, 128, 128, fp32=True) == (32, 128, 16, 16, 16, 12)
    assert cfg(4194304, 32, 64, 64, 16, fp32=True) == (32, 16, 16, 16, 16, 12)
    assert cfg(1048576, 64, 64, 64, 64, fp32=True) == (32, 64, 16, 16, 16, 12)
    assert kernel._mirror_policy(4096, (128,) * 6, 256, fp32=True) == (32, 4)  # 5 layers: one group
    assert callable(kernel._fused_mlp_fwd) and kernel.Model and kernel.ModelNew


def test_model_reference_matches_oracle_on_cpu():
    # kernel.Model is the eager reference (kernel.py:163-171); on the CPU in
    # fp32 it must agree with the oracle.
    import numpy as np

    import kernel
    from oracle import mlp_oracle as orc

    x, ws = orc.make_inputs((128, 128, 128, 128), 64, seed=0)
    got = kernel.Model()(*[torch.from_numpy(a.astype(np.float32)) for a in [x] + ws]).numpy()
    np.testing.assert_allclose(got, orc.forward(x, ws), rtol=1e-4, atol=1e-5)


def test_launch_shim_converts_arguments_like_ctypes():
    # The CPython shims (csrc/pylaunch.c) call the entry points of the library
    # ctypes loaded; argument validation answers exactly as through ctypes.
    shim = ops._fast()
    if shim is None:
        pytest.skip("the _mlpmk_launch module is not built")
    d = (128, 128, 128, 128)
    w, dw, st = (A, A, A), (A, A, A), (A, A)
    assert shim.fwd(d, 99, A, w, A, None, 256, None) == INVALID  # bad dtype
    assert shim.fwd(d, 1, A, w, A, None, -1, None) == INVALID  # negative M
    assert shim.bwd(d, 1, A, w, st, A, -2, None, dw, None, 0, 256, None) == INVALID  # bad dout stride
    assert shim.bwd(d, 1, A, w, st, A + 1, -1, None, dw, None, 0, 256, None) == MISALIGNED
    if ops.bwd_supported(list(d)):
        assert shim.bwd(d, 1, A, w, st, A, 128, None, dw, None, 0, 0, None) == OK  # M = 0: nothing to do
    with pytest.raises(ValueError):
        shim.fwd(d, 1, A, (A, A), A, None, 256, None)  # one weight short
    with pytest.raises(TypeError):
        shim.fwd(list(d), 1, A, w, A, None, 256, None)  # dims must be a tuple
    with pytest.raises(TypeError):
        shim.fwd(d, 1, A, w, A, None, 256)  # stream missing
