"""The reference's large-M backward fallback, on MI355X.

/root/reference/mlp_fused.md:114-146: above an M threshold the reference
leaves its fused Triton backward (whose fp32 weight-gradient atomics contend)
for library GEMMs plus one fused elementwise kernel, ``sigmoid_h_mul``
(``dz = (1 - exp(-h)) * dh``), with the weight-gradient GEMM of each layer
issued right after that layer's data-gradient GEMM ("interleaved", so that
h_l and dz_l are still in L2):

    dh2 = grad @ W3.T  ->  dw3 = h2.T @ grad
    dz2 = sigmoid(h2) * dh2  ->  dh1 = dz2 @ W2.T
    dw2 = h1.T @ dz2 ...

Here the GEMMs are rocBLAS / hipBLASLt calls through torch (data gradients in
the 16-bit element type with fp32 accumulation, weight gradients in fp32 from
the fp32 stash: sums over many rows would overflow fp16) and the elementwise
step is this library's ``mlpmk_sigmoid_h_mul`` HIP kernel, which writes dz in
fp32 for the weight-gradient GEMM and in the 16-bit type for the next
data-gradient GEMM from one read of h and dh.

The fused backward megakernel (``ops.bwd``) replaces this at every M on
MI355X -- it needs no atomics in its workspace form and was measured 4.6-21x
faster at M = 4K..1M -- so autograd uses it unless ``autograd.BACKWARD`` is
set to ``"fallback"``; this path is kept as the reference's alternative and as
a comparator.  Same arguments and results as ``ops.bwd``.

For networks no fused forward takes (fp32 tensors wider than 128, any
tensors wider than 256 or deeper than 5 layers), :func:`fwd` is the matching
forward: fp32 library GEMMs and this library's fp32 softplus kernel
(``mlpmk_softplus_f32``); :func:`bwd` then runs the backward (every GEMM in
fp32 for fp32 tensors).
"""
from __future__ import annotations

import torch

from . import _lib
from .ops import _check, _elem_code, _launch


def sigmoid_h_mul(h, dh, dz16_dtype=None):
    """``dz = dh * (1 - exp(-h))`` (``mlpmk_sigmoid_h_mul``): ``h`` fp32, ``dh``
    fp32 / fp16 / bf16, same shape, contiguous, on one GPU.  Returns the fp32
    ``dz`` and, when ``dz16_dtype`` is given, ``dz`` in that 16-bit type."""
    if h.dtype != torch.float32 or h.shape != dh.shape:
        raise ValueError("h must be fp32 and shaped like dh")
    if not (h.is_contiguous() and dh.is_contiguous()) or h.device != dh.device or h.device.type != "cuda":
        raise ValueError("h and dh must be contiguous tensors on one GPU")
    dh_code = _lib.DTYPE_F32 if dh.dtype == torch.float32 else _elem_code(dh.dtype, "dh")
    dz32 = torch.empty_like(h)
    dz16 = torch.empty_like(h, dtype=dz16_dtype) if dz16_dtype is not None else None
    dz16_code = _elem_code(dz16_dtype, "dz16") if dz16_dtype is not None else _lib.DTYPE_F16
    lib = _lib.get()
    rc = _launch(h.device, lib.mlpmk_sigmoid_h_mul, h.data_ptr(), dh.data_ptr(), dh_code, dz32.data_ptr(),
                 dz16.data_ptr() if dz16 is not None else None, dz16_code, h.numel())
    _check("mlpmk_sigmoid_h_mul", rc)
    return (dz32, dz16) if dz16_dtype is not None else dz32


def softplus_f32(z, out=None):
    """``h = softplus(z)`` elementwise in fp32 (``mlpmk_softplus_f32``: torch's
    softplus with beta 1 and threshold 20, kernel.py:168-171).  ``z`` fp32,
    contiguous, on a GPU; ``out`` may be ``z`` itself (default: a new tensor)."""
    if z.dtype != torch.float32 or not z.is_contiguous() or z.device.type != "cuda":
        raise ValueError("z must be a contiguous fp32 tensor on a GPU")
    h = torch.empty_like(z) if out is None else out
    if h.shape != z.shape or h.dtype != torch.float32 or not h.is_contiguous() or h.device != z.device:
        raise ValueError("out must be a contiguous fp32 tensor shaped like z on its GPU")
    rc = _launch(z.device, _lib.get().mlpmk_softplus_f32, z.data_ptr(), h.data_ptr(), z.numel())
    _check("mlpmk_softplus_f32", rc)
    return h


def fwd(x, weights, stash=False):
    """Forward layer by layer, for the networks no fused forward takes: fp32
    tensors wider than 128, any tensors wider than 256, more than 5 layers,
    hidden widths that are not multiples of 16.  ``z = a @ W_l``
    as an fp32 library GEMM (rocBLAS / hipBLASLt through torch; 16-bit
    values are exact in fp32, so this is the fused kernels' fp32
    accumulation), then the fp32 softplus kernel on every hidden layer, whose
    output is rounded to the tensor format before the next GEMM as the
    reference's kernel rounds its h (kernel.py:110,117).  The reference's
    kernels take any width (kernel.py:60-63; INPUT_DTYPE = fp32,
    mlp_fused.md:159-166).  Returns ``out`` in x's dtype, or ``(out, [h1 ..
    h_{L-1}])`` with the fp32 stash that :func:`bwd` reads."""
    dt = x.dtype
    if dt not in (torch.float32, torch.float16, torch.bfloat16) or any(w.dtype != dt for w in weights):
        raise ValueError("x and the weights must share one of fp32, fp16 or bf16")
    a = x.contiguous() if dt == torch.float32 else x.float()
    hs = []
    with torch.autocast("cuda", enabled=False):  # the GEMMs stay fp32 under a caller's autocast
        for i, w in enumerate(weights):
            z = a @ (w.contiguous() if dt == torch.float32 else w.float())
            if i + 1 < len(weights):
                h = softplus_f32(z, out=z)
                hs.append(h)
                a = h if dt == torch.float32 else h.to(dt).float()
            else:
                a = z if dt == torch.float32 else z.to(dt)
    return (a, hs) if stash else a


def bwd(x, weights, hs, dout, dws, dx=None):
    """Gradients of ``out = MLP(x)`` from the fp32 stash ``hs`` = [h1 ..
    h_{L-1}]: ``dws[l] += h_l^T dz_l`` (``h_0 = x``) and, if ``dx`` is given,
    ``dx = dz_0 W_0^T``, in the interleaved order of mlp_fused.md:139-145.
    ``dout`` may be a broadcast row (stride 0), as ``loss = out.sum()``
    gives."""
    L = len(weights)
    if len(hs) != L - 1 or any(h is None for h in hs):
        raise ValueError("the fallback backward reads every hidden activation from the stash (no recompute)")
    with torch.autocast("cuda", enabled=False):  # GEMMs in the types below, whatever the caller's autocast
        return _bwd(x, weights, hs, dout, dws, dx)


def _bwd(x, weights, hs, dout, dws, dx):
    L = len(weights)
    dt = x.dtype
    dz16 = dout.to(dt).contiguous() if dout.stride(0) != 0 else dout[:1].to(dt).expand_as(dout).contiguous()
    dz32 = dz16.float()
    f32 = dt == torch.float32  # fp32 tensors: every GEMM in fp32
    for l in range(L - 1, -1, -1):
        need_dh = l > 0 or dx is not None
        if need_dh:
            dh = dz16 @ weights[l].t().contiguous()  # data gradient: 16-bit GEMM, fp32 accumulation
        a = hs[l - 1] if l > 0 else x.float()
        dws[l].add_(a.t() @ dz32)  # weight gradient: fp32 GEMM, right after (interleaved)
        if l > 0 and f32:
            dz32 = dz16 = sigmoid_h_mul(hs[l - 1], dh.contiguous())
        elif l > 0:
            dz32, dz16 = sigmoid_h_mul(hs[l - 1], dh.contiguous(), dz16_dtype=dt)
        elif dx is not None:
            dx.copy_(dh)
    return dws, dx
