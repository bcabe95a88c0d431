"""``torch.autograd.Function`` wrappers of the megakernels.

Training path of the reference's ``FusedMLPSoftplus`` / ``FusedMLPSoftplusWN``
(/root/reference/README.md:18,24-34,58-70; /root/reference/mlp_fused.md:52-61,
80-112,159-172,461-486 -- ``fused_mlp.py`` itself is not in the snapshot):

* forward: one forward-megakernel launch that also writes the fp32 activation
  stash (``mlpmk_fwd`` with ``stash``); with weight norm, one weight-norm launch
  for all layers first (``mlpmk_wn_fwd``).
* backward: one backward-megakernel launch (``mlpmk_bwd``) producing every fp32
  weight gradient (and ``dx`` when ``x`` needs it); with weight norm, one more
  launch turning all ``dW`` into ``dv, dg`` (``mlpmk_wn_bwd``).
* activation recomputation (``RECOMPUTE``): for networks with a recomputing
  backward (``ops.bwd_recompute_supported``) and ``x`` without grad, the
  forward stashes h_1 .. h_{L-2} only and the backward recomputes h_{L-1}
  (/root/reference/mlp_fused.md:451-452 lists this trade as future work).
* AMP: ``custom_fwd`` / ``custom_bwd`` as mlp_fused.md:168-172 describes.
  The reference casts to fp16 (``cast_inputs=torch.float16``); here the
  tensors take the autocast dtype, so ``torch.autocast(dtype=torch.bfloat16)``
  runs the bf16 kernels and fp16 autocast the fp16 ones (``kernel_dtype``).
  Outside autocast the tensors keep their own type, as the reference's
  INPUT_DTYPE kernels do (mlp_fused.md:159-166): fp32 parameters and an fp32
  ``x`` run the fp32-tensor kernels (bf16 hi/lo split operands: fp32's
  exponent range) and return an fp32 ``out``.  Networks no fused forward
  takes (fp32 ones wider than 128, any wider than 256) run layer by layer
  (``fallback.fwd``: fp32 library GEMMs, the library's fp32 softplus kernel,
  hidden values rounded to the tensor format between layers) and train
  through the fallback backward.
* inference: ``fused_mlp`` / ``fused_mlp_wn`` (and the modules) call the plain
  forward, without the fp32 stash, whenever autograd will not need it -- grad
  disabled (``torch.no_grad`` / ``inference_mode``) or nothing requiring grad.
  Inside ``Function.forward`` grad mode is always off and
  ``ctx.needs_input_grad`` reflects ``requires_grad`` only, so that choice is
  made before ``apply``.

Every kernel of the fused paths is ``libmlpmk.so``'s and there is no CPU
path; the layer-by-layer fp32 forward and the fallback backward issue their
GEMMs as library GEMMs (rocBLAS / hipBLASLt through torch) around the
library's elementwise kernels.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from . import _lib, ops

# Activation recomputation policy: "auto" recomputes h_{L-1} where that makes
# the training step faster (MI355X, stash -> recompute; the weight-norm
# module's step replayed as one HIP graph, or forward + backward with dx):
# 3 layers from RECOMPUTE_MIN_ROWS rows (0.137 -> 0.140 ms at 131072 rows,
# 0.239 -> 0.223 ms at 262144, 0.782 -> 0.726 ms at 1048576; with dx 118 ->
# 125 us at 131072 rows, 229 -> 227 us at 262144, 785 -> 779 us at
# 1048576), 5 layers from
# RECOMPUTE_MIN_ROWS_5L (0.256 -> 0.253 ms at 131072 rows, 1.481 -> 1.379 ms
# at 1048576; with dx 221 -> 211 us at 131072).  "always" / "never" force
# the choice where the shape allows it.
RECOMPUTE = "auto"
RECOMPUTE_MIN_ROWS = 1 << 18
RECOMPUTE_MIN_ROWS_5L = 1 << 17

# Backward implementation: "fused" (the backward megakernel, every M) or
# "fallback" (the reference's large-M path of library GEMMs and the fused
# sigmoid_h_mul kernel, mlp_fused.md:114-146; mlpmk.fallback).  The fallback
# reads every activation from the stash, so it turns recomputation off.
BACKWARD = "fused"

_rc_shapes = {}


def _backward_impl():
    if BACKWARD not in ("fused", "fallback"):
        raise ValueError(f"BACKWARD must be 'fused' or 'fallback', got {BACKWARD!r}")
    return BACKWARD


_bwd_shapes = {}


def _fused_bwd_supported(dims, dtype=torch.float16):
    key = (dims, dtype)
    ok = _bwd_shapes.get(key)
    if ok is None:
        ok = _bwd_shapes[key] = ops.bwd_supported(list(dims), dtype)
    return ok


def _run_bwd(x, weights, hs, dout, dws, dx):
    # Shapes without a fused backward (output widths that are not a multiple
    # of 8 above 128, or fp32 ones not a multiple of 8) take the fallback:
    # the reference's own route for shapes its fused kernel does not cover.
    dims = tuple([int(x.shape[1])] + [int(w.shape[1]) for w in weights])
    if _backward_impl() == "fallback" or not _fused_bwd_supported(dims, x.dtype):
        from . import fallback

        fallback.bwd(x, weights, hs, dout, dws, dx)
    else:
        ops.bwd(x, weights, hs, dout, dws, dx)


def _use_recompute(dims, m, need_dx, dtype=torch.float16):
    if RECOMPUTE == "never" or _backward_impl() == "fallback" or not _fused_bwd_supported(tuple(dims), dtype):
        return False
    if dtype == torch.float32:  # (the recomputing kernels are 16-bit ones)
        return False
    if RECOMPUTE not in ("auto", "always"):
        raise ValueError(f"RECOMPUTE must be 'auto', 'always' or 'never', got {RECOMPUTE!r}")
    ok = _rc_shapes.get(dims)
    if ok is None:
        ok = _rc_shapes[dims] = ops.bwd_recompute_supported(list(dims))
    if RECOMPUTE == "always" or not ok:
        return ok
    del need_dx  # (the recomputing backward also writes dx)
    return m >= (RECOMPUTE_MIN_ROWS_5L if len(dims) == 6 else RECOMPUTE_MIN_ROWS)


def kernel_dtype(x, dims=None):
    """Element type the network runs in for input ``x``: the autocast dtype
    when autocast is on (fp16 unless it is bf16); else ``x``'s own type --
    bf16, fp16 or fp32 (the fp32-tensor kernels for widths up to 128, the
    layer-by-layer fp32 path of ``mlpmk.fallback`` above) --, fp32 for
    float64 (the widest type the library computes in: the range stays), and
    fp16 for anything else.  ``dims`` is accepted for the callers'
    convenience."""
    del dims
    if torch.is_autocast_enabled("cuda"):
        return torch.bfloat16 if torch.get_autocast_dtype("cuda") == torch.bfloat16 else torch.float16
    if x.dtype in (torch.bfloat16, torch.float32):
        return x.dtype
    if x.dtype == torch.float64:
        return torch.float32
    return torch.float16


_fwd_shapes = {}


def _layerwise(dims, dtype):
    """True when no fused forward takes ``dims`` for ``dtype`` tensors (fp32
    networks wider than 128, any network wider than 256 or deeper than the
    kernels' 5 layers): they run layer by layer (``fallback.fwd``: fp32
    library GEMMs and the library's fp32 softplus kernel)."""
    key = (tuple(dims), dtype)
    ok = _fwd_shapes.get(key)
    if ok is None:
        ok = _fwd_shapes[key] = ops.fwd_supported(list(key[0]), dtype)
    return not ok


def _input_pad(dims, dtype):
    """Zero columns to append to ``x`` (and zero rows to W_1) so that a
    fused forward takes the network: input widths that are not multiples of
    16 (e.g. the 3 coordinates of a neural field) where the padded network
    is otherwise a fused one; 0 if none is needed or none helps.  The
    padding adds nothing to any product; dx and dW_1 drop it again."""
    d0 = dims[0]
    if d0 % 16 == 0:
        return 0
    pad = -d0 % 16
    return 0 if _layerwise((d0 + pad,) + tuple(dims[1:]), dtype) else pad


def _padded(x, w0, pad):
    """``x`` with ``pad`` zero columns and ``w0`` with ``pad`` zero rows."""
    return F.pad(x, (0, pad)), F.pad(w0, (0, 0, 0, pad))


def _needs_graph(*tensors):
    """True when autograd will run a backward through this call."""
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _as_row_broadcast(dout):
    """``dout`` with unit column stride, keeping a broadcast row (stride 0)
    as a broadcast and a fully expanded scalar (strides (0, 0): what ``loss =
    out.sum()`` hands back) as it is -- the backward kernels read that one
    element for every row and column."""
    if dout.dim() == 2 and (dout.stride(1) == 1 or dout.stride() == (0, 0)):
        return dout
    m, n = dout.shape
    if dout.stride(0) == 0:
        return dout[:1].contiguous().expand(m, n)
    return dout.contiguous()


class FusedMLPFunction(torch.autograd.Function):
    """``out = softplus(... softplus(x @ W1) ...) @ WL`` with the fused backward.

    Inputs: ``x`` [M, D] and L weights [in, out], cast to ``kernel_dtype(x)``
    (autograd casts the gradients back).  Returns ``out`` [M, OUT] of that
    dtype.  Always writes the stash when some input requires grad; use
    ``fused_mlp`` to skip it when grad is disabled.
    """

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x, *weights):
        dims = (int(x.shape[1]),) + tuple(int(w.shape[1]) for w in weights)
        dt = kernel_dtype(x, dims)
        x = x.to(dt).contiguous()
        weights = [w.to(dt).contiguous() for w in weights]
        pad = _input_pad(dims, dt)
        if pad:
            x, w0 = _padded(x, weights[0], pad)
            weights = [w0] + weights[1:]
            dims = (dims[0] + pad,) + dims[1:]
        if any(ctx.needs_input_grad):
            rc = _use_recompute(dims, int(x.shape[0]), ctx.needs_input_grad[0], dt)
            if _layerwise(dims, dt):
                from . import fallback

                out, hs = fallback.fwd(x, weights, stash=True)
            else:
                out, hs = ops.fwd(x, weights, stash=True, recompute=rc)
            ctx.save_for_backward(x, *weights, *[h for h in hs if h is not None])
            ctx.dims = dims
            ctx.recompute = rc
            ctx.pad = pad
        elif _layerwise(dims, dt):
            from . import fallback

            out = fallback.fwd(x, weights)
        else:
            out = ops.fwd(x, weights)
        return out

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    @once_differentiable  # the library's gradients carry no graph: a second derivative raises
    def backward(ctx, dout):
        dims = ctx.dims
        L = len(dims) - 1
        saved = ctx.saved_tensors
        x, weights, hs = saved[0], list(saved[1 : 1 + L]), list(saved[1 + L :])
        if ctx.recompute:
            hs.append(None)  # h_{L-1}: recomputed by the backward kernel
        dout = _as_row_broadcast(dout.to(x.dtype))
        dx = torch.empty_like(x) if ctx.needs_input_grad[0] else None
        if _backward_impl() == "fused" and _fused_bwd_supported(dims, x.dtype):
            # x, the weights and the stash were checked by the forward.  The
            # library writes dW (MLPMK_BWD_WRITE_DW): no zero-fill launch.
            dws = [torch.empty(w.shape, dtype=torch.float32, device=w.device) for w in weights]
            M = int(x.shape[0])
            dout, row_stride = ops._dout_rows(dout, M, dims[-1], x.dtype, x.device)
            ops._bwd_raw(x.device, dims, ops._fwd_code(x.dtype) | _lib.BWD_WRITE_DW, x.data_ptr(),
                         [w.data_ptr() for w in weights], [h.data_ptr() if h is not None else None for h in hs],
                         dout.data_ptr(), row_stride, dx.data_ptr() if dx is not None else None,
                         [d.data_ptr() for d in dws], M)
        else:
            dws = [torch.zeros(w.shape, dtype=torch.float32, device=w.device) for w in weights]
            _run_bwd(x, weights, hs, dout, dws, dx)
        if ctx.pad:  # drop the zero columns of x (rows of W_1) the forward appended
            d0 = dims[0] - ctx.pad
            dx = dx[:, :d0] if dx is not None else None
            dws[0] = dws[0][:d0]
        return (dx, *[d if need else None for d, need in zip(dws, ctx.needs_input_grad[1:])])


class FusedMLPWNFunction(torch.autograd.Function):
    """Weight-normalised MLP: ``W_l[:, j] = g_l[j] v_l[:, j] / ||v_l[:, j]||``
    for every layer from the contiguous blocks ``v_all`` / ``g_all``
    (mlp_fused.md:478-480), then the fused MLP.

    Launches: forward = weight norm (all layers) + forward megakernel;
    backward = backward megakernel + weight-norm backward (all layers).
    The buffers between them (W, 1/||v||, the stash, dW, dv, dg) are
    allocated here with known shapes, so the launches take their pointers
    directly (``ops._*_raw``) instead of per-layer views.
    """

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x, v_all, g_all, dims):
        dims = tuple(int(d) for d in dims)
        x = x.to(kernel_dtype(x, dims)).contiguous()
        nw, ng, woff = _layout(dims)
        dev = x.device
        if dev.type != "cuda":
            raise ValueError(f"x must be on a GPU device, got {dev}")
        if x.dim() != 2 or int(x.shape[1]) != dims[0]:
            raise ValueError(f"x has shape {tuple(x.shape)}, expected [M, {dims[0]}]")
        v_all = v_all.contiguous()
        g_all = g_all.contiguous()
        pcode = ops._param_dtype(v_all)
        if g_all.dtype != v_all.dtype or v_all.device != dev or g_all.device != dev:
            raise TypeError("v_all and g_all must share a dtype and x's device")
        if v_all.numel() != nw or g_all.numel() != ng:
            raise ValueError("weight-norm block sizes do not match dims")
        code = ops._fwd_code(x.dtype)
        w_all = torch.empty(nw, dtype=x.dtype, device=dev)  # the megakernels' element type
        inv_all = torch.empty(ng, dtype=torch.float32, device=dev)
        ops._wn_fwd_raw(dev, dims, pcode, code, v_all.data_ptr(), g_all.data_ptr(), w_all.data_ptr(),
                        inv_all.data_ptr())
        wb, es = w_all.data_ptr(), w_all.element_size()
        w_ptrs = [wb + es * o for o in woff]
        M = int(x.shape[0])
        ctx.pad = pad = _input_pad(dims, x.dtype)
        if pad:
            # Input width padded to a multiple of 16 (zero columns of x, zero
            # rows of W_1) so that the fused kernels take the network.
            ws = _split(w_all, dims)
            xp, w0 = _padded(x, ws[0], pad)
            ws = [w0] + ws[1:]
            if any(ctx.needs_input_grad):
                pdims = (dims[0] + pad,) + dims[1:]
                rc = _use_recompute(pdims, M, ctx.needs_input_grad[0], x.dtype)
                out, hs = ops.fwd(xp, ws, stash=True, recompute=rc)
                ctx.save_for_backward(xp, v_all, g_all, w_all, inv_all, *[h for h in hs if h is not None])
                ctx.dims = dims
                ctx.recompute = rc
                return out
            return ops.fwd(xp, ws)
        if _layerwise(dims, x.dtype):
            from . import fallback

            if any(ctx.needs_input_grad):
                out, hs = fallback.fwd(x, _split(w_all, dims), stash=True)
                ctx.save_for_backward(x, v_all, g_all, w_all, inv_all, *hs)
                ctx.dims = dims
                ctx.recompute = False
                return out
            return fallback.fwd(x, _split(w_all, dims))
        out = torch.empty((M, dims[-1]), dtype=x.dtype, device=dev)
        if any(ctx.needs_input_grad):
            rc = _use_recompute(dims, M, ctx.needs_input_grad[0], x.dtype)
            hs = [torch.empty((M, d), dtype=torch.float32, device=dev) for d in dims[1:-1]]
            if rc:
                hs[-1] = None
            ops._fwd_raw(dev, dims, code, x.data_ptr(), w_ptrs, out.data_ptr(),
                         [h.data_ptr() if h is not None else None for h in hs], M)
            ctx.save_for_backward(x, v_all, g_all, w_all, inv_all, *[h for h in hs if h is not None])
            ctx.dims = dims
            ctx.recompute = rc
        else:
            ops._fwd_raw(dev, dims, code, x.data_ptr(), w_ptrs, out.data_ptr(), None, M)
        return out

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    @once_differentiable  # the library's gradients carry no graph: a second derivative raises
    def backward(ctx, dout):
        dims = ctx.dims
        nw, ng, woff = _layout(dims)
        x, v_all, g_all, w_all, inv_all, *hs = ctx.saved_tensors
        if ctx.recompute:
            hs.append(None)  # h_{L-1}: recomputed by the backward kernel
        dev = x.device
        M = int(x.shape[0])
        dout = _as_row_broadcast(dout.to(x.dtype))
        dx = torch.empty_like(x) if ctx.needs_input_grad[0] else None
        if ctx.pad:
            # x was saved padded: W_1 padded the same way, dW_1 computed padded
            # and its first rows copied into the flat block, dx cut back.
            pdims = (dims[0] + ctx.pad,) + dims[1:]
            ws = _split(w_all, dims)
            ws = [F.pad(ws[0], (0, 0, 0, ctx.pad))] + ws[1:]
            dw_all = torch.empty(nw, dtype=torch.float32, device=dev)
            dws = _split(dw_all, dims)
            dw0 = torch.empty((pdims[0], dims[1]), dtype=torch.float32, device=dev)
            if _backward_impl() == "fused" and _fused_bwd_supported(pdims, x.dtype):
                ops.bwd(x, ws, hs, dout, [dw0] + dws[1:], dx, accumulate=False)
            else:
                dw0.zero_()
                for d in dws[1:]:
                    d.zero_()
                _run_bwd(x, ws, hs, dout, [dw0] + dws[1:], dx)
            dws[0].copy_(dw0[: dims[0]])
            if dx is not None:
                dx = dx[:, : dims[0]]
        elif _backward_impl() == "fused" and _fused_bwd_supported(dims, x.dtype):
            # dW written by the library (MLPMK_BWD_WRITE_DW): no zero-fill launch.
            dw_all = torch.empty(nw, dtype=torch.float32, device=dev)
            dout, row_stride = ops._dout_rows(dout, M, dims[-1], x.dtype, dev)
            wb, gb, es = w_all.data_ptr(), dw_all.data_ptr(), w_all.element_size()
            ops._bwd_raw(dev, dims, ops._fwd_code(x.dtype) | _lib.BWD_WRITE_DW, x.data_ptr(),
                         [wb + es * o for o in woff], [h.data_ptr() if h is not None else None for h in hs],
                         dout.data_ptr(), row_stride, dx.data_ptr() if dx is not None else None,
                         [gb + 4 * o for o in woff], M)
        else:
            dw_all = torch.zeros(nw, dtype=torch.float32, device=dev)
            _run_bwd(x, _split(w_all, dims), hs, dout, _split(dw_all, dims), dx)
        dv = dg = None
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            dv = torch.empty_like(v_all)
            dg = torch.empty_like(g_all)
            ops._wn_bwd_raw(dev, dims, ops._param_dtype(v_all), dw_all.data_ptr(), v_all.data_ptr(),
                            g_all.data_ptr(), inv_all.data_ptr(), dv.data_ptr(), dg.data_ptr())
        return dx, dv, dg, None


_layouts = {}


def _layout(dims):
    """``(n_weights, n_columns, element offsets of each W_l)`` of the flat
    weight-norm blocks of ``dims`` (cached)."""
    lay = _layouts.get(dims)
    if lay is None:
        offs, o = [], 0
        for i in range(len(dims) - 1):
            offs.append(o)
            o += dims[i] * dims[i + 1]
        lay = _layouts[dims] = (o, sum(dims[1:]), tuple(offs))
    return lay


def _split(flat, dims):
    """Views of the per-layer [in, out] blocks of a flat parameter block."""
    out, off = [], 0
    for i in range(len(dims) - 1):
        n = dims[i] * dims[i + 1]
        out.append(flat[off : off + n].view(dims[i], dims[i + 1]))
        off += n
    return out


def fused_mlp(x, *weights):
    """Functional form of :class:`FusedMLPFunction`: the training forward
    (with the fp32 stash) when autograd will need it, else one plain forward
    launch."""
    if _needs_graph(x, *weights):
        return FusedMLPFunction.apply(x, *weights)
    dims = (int(x.shape[1]),) + tuple(int(w.shape[1]) for w in weights)
    dt = kernel_dtype(x, dims)
    x = x.to(dt).contiguous()
    weights = [w.to(dt).contiguous() for w in weights]
    pad = _input_pad(dims, dt)
    if pad:
        x, w0 = _padded(x, weights[0], pad)
        return ops.fwd(x, [w0] + weights[1:])
    if _layerwise(dims, dt):
        from . import fallback

        return fallback.fwd(x, weights)
    return ops.fwd(x, weights)


def fused_mlp_wn(x, v_all, g_all, dims):
    """Functional form of :class:`FusedMLPWNFunction` (same stash rule as
    :func:`fused_mlp`)."""
    dims = tuple(int(d) for d in dims)
    if _needs_graph(x, v_all, g_all):
        return FusedMLPWNFunction.apply(x, v_all, g_all, dims)
    x = x.to(kernel_dtype(x, dims)).contiguous()
    w_all = torch.empty(sum(dims[i] * dims[i + 1] for i in range(len(dims) - 1)), dtype=x.dtype, device=x.device)
    inv_all = torch.empty(sum(dims[1:]), dtype=torch.float32, device=x.device)
    ops.wn_fwd(dims, v_all.contiguous(), g_all.contiguous(), w_all, inv_all)
    pad = _input_pad(dims, x.dtype)
    if pad:
        ws = _split(w_all, dims)
        xp, w0 = _padded(x, ws[0], pad)
        return ops.fwd(xp, [w0] + ws[1:])
    if _layerwise(dims, x.dtype):
        from . import fallback

        return fallback.fwd(x, _split(w_all, dims))
    return ops.fwd(x, _split(w_all, dims))
