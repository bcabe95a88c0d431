"""fp32 tensors through the forward and the backward (``mlpmk_fwd`` /
``mlpmk_bwd_ws`` with MLPMK_DTYPE_F32, the drop-in ``kernel._fused_mlp_fwd``
and the modules outside autocast).  The reference's launcher passes fp32
``x`` on (/root/reference/kernel.py:130-138) and its kernels take fp32
tensors through INPUT_DTYPE (/root/reference/mlp_fused.md:159-166), where
``tl.dot`` rounds the operands to TF32 (10-bit significand, fp32 exponent
range).  Here every MFMA operand is split into bf16 hi + lo (products hi*hi
+ hi*lo + lo*hi): fp32's exponent range and a ~16-bit significand, with fp32
accumulation, softplus, stash, outputs and data gradients.

Checks, against the oracle evaluated in float64 on the same fp32 values:
outputs at atol = rtol = 2e-4 of the row's scale (the fp16 path's bound is
1e-2), weight gradients per entry within 1e-3 |ref| + 1e-4 max|ref| and
relative Frobenius 5e-4, dx at atol = rtol = 2e-4 of its row scale.  Rows
far outside fp16's range (|x| up to 1e6 and 1e30, and down to 1e-12) keep
those bounds: fp32's exponent range end to end.
"""
import numpy as np
import pytest
import torch

import kernel
from mlpmk import ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-4

SHAPES = [
    ((128, 128, 128, 128), 4096),
    ((128, 128, 128, 128), 131072),
    ((128,) * 6, 16384),
    ((32, 64, 64, 16), 4096),
    ((64, 96, 48, 10), 3001),        # runtime widths, ragged M, output width not a multiple of 8
    ((48, 128, 32), 1000),           # 2 layers
    ((128, 112, 96, 80, 3), 777),    # 4 layers
    ((16, 32, 48, 64, 80, 128), 257),  # 5 layers, runtime widths
]


def _inputs(dims, m, seed, wide_rows=False):
    """fp32 x and weights with full fp32 significands (not 16-bit values);
    with wide_rows, every 7th row scaled by 1e6, every 11th by 1e-12 and row 3
    by 1e30 -- far outside fp16's range either way."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, dims[0])).astype(np.float32)
    ws = [(rng.standard_normal((dims[i], dims[i + 1])) / np.sqrt(dims[i])).astype(np.float32)
          for i in range(len(dims) - 1)]
    if wide_rows and m > 3:
        x[::7] *= np.float32(1e6)
        x[::11] *= np.float32(1e-12)
        x[3] *= np.float32(1e30)
    return x, ws


def _check_rows(got, ref, what, tol=TOL):
    """|got - ref| <= tol |ref| + tol max_row |ref| (every row on its own scale)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max(axis=1, keepdims=True)
    err = np.abs(got - ref)
    excess = err - (tol * np.abs(ref) + tol * scale)
    assert np.all(np.isfinite(got)), f"{what}: non-finite outputs"
    assert excess.max() <= 0, f"{what}: worst excess {excess.max():.3g} (max rel err {(err / np.maximum(scale, 1e-300)).max():.3g})"


def _run(x, ws, stash=False):
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    return ops.fwd(xd, wd, stash=stash)


@pytest.mark.parametrize("dims,m", SHAPES)
def test_fp32_forward_matches_oracle(dims, m):
    x, ws = _inputs(dims, m, seed=len(dims) * 1000 + m)
    out = _run(x, ws)
    assert out.dtype == torch.float32 and tuple(out.shape) == (m, dims[-1])
    _check_rows(out.cpu().numpy(), orc.forward(x, ws, dtype=np.float64), f"fp32 {dims} M={m}")


@pytest.mark.parametrize("dims,m", [((128, 128, 128, 128), 4096), ((64, 96, 48, 10), 3001), ((128,) * 6, 1000)])
def test_fp32_forward_keeps_the_fp32_range(dims, m):
    # |x| up to 1e30 (fp16 overflows past 65,504) and down to 1e-12 (below
    # fp16's subnormals): every row within the same relative bound.  Hidden
    # pre-activations of the large rows pass z > 88.7, where 2^u overflows
    # and softplus(z) = z is taken.
    x, ws = _inputs(dims, m, seed=5 + m, wide_rows=True)
    out, hs = _run(x, ws, stash=True)
    ref, ref_h = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    assert np.abs(ref).max() > 1e28
    _check_rows(out.cpu().numpy(), ref, f"fp32 range {dims} M={m}")
    for i, (h, rh) in enumerate(zip(hs, ref_h)):
        _check_rows(h.cpu().numpy(), rh, f"stash h{i + 1}")


def test_fp32_stash_matches_oracle_hidden():
    dims, m = (128, 128, 128, 128), 8192
    x, ws = _inputs(dims, m, seed=3)
    out, hs = _run(x, ws, stash=True)
    ref, ref_h = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    _check_rows(out.cpu().numpy(), ref, "out")
    for i, (h, rh) in enumerate(zip(hs, ref_h)):
        _check_rows(h.cpu().numpy(), rh, f"h{i + 1}")
    # inference and training forward write the same output bits
    assert torch.equal(_run(x, ws), out)


@pytest.mark.parametrize("xview,wview", [("contiguous", "contiguous"), ("transposed", "sliced")])
def test_fp32_launcher_matches_model_and_oracle(xview, wview):
    dims, m = (128, 128, 128, 128), 4096
    x, ws = _inputs(dims, m, seed=21)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    if xview == "transposed":
        xd = xd.t().contiguous().t()  # same values, column-major storage
    if wview == "sliced":
        wd = [torch.cat([w, w], dim=1)[:, : w.shape[1]] for w in wd]  # non-contiguous views
    out = kernel._fused_mlp_fwd(xd, *wd)
    assert out.dtype == torch.float32
    _check_rows(out.cpu().numpy(), orc.forward(x, ws, dtype=np.float64), "launcher vs oracle")
    eager = kernel.Model()(xd, *wd)  # the reference's eager fp32 model on the GPU
    ok, err, _ = orc.allclose_report(out.cpu().numpy(), eager.cpu().numpy(), 1e-2, 1e-2)
    assert ok, err
    assert torch.equal(kernel.ModelNew()(xd, *wd), out)


def test_fp32_small_and_empty_batches():
    dims = (128, 128, 128, 128)
    for m in (0, 1, 31, 33, 255):
        x, ws = _inputs(dims, m, seed=m)
        out = _run(x, ws)
        assert tuple(out.shape) == (m, 128)
        if m:
            _check_rows(out.cpu().numpy(), orc.forward(x, ws, dtype=np.float64), f"M={m}")


def test_mixed_dtypes_are_rejected():
    x = torch.zeros((64, 128), device="cuda", dtype=torch.float32)
    ws = [torch.zeros((128, 128), device="cuda", dtype=torch.float16) for _ in range(3)]
    with pytest.raises(TypeError):
        ops.fwd(x, ws)


# ---------------------------------------------------------------------------
# Backward with fp32 tensors (the two-pass backward, bf16 hi/lo operands)
# ---------------------------------------------------------------------------

def _check_dw32(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    worst = np.max(np.abs(got - ref) - (1e-3 * np.abs(ref) + 1e-4 * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300)
    assert worst <= 0 and frob < 5e-4, f"{what}: worst excess {worst:.3g} (scale {scale:.3g}), rel frob {frob:.3g}"


def _train32(dims, m, seed, dout_mode, with_dx, wide_rows=False, own_stash=False):
    """The fp32 backward against the oracle's float64 backward.  With
    own_stash the oracle is fed the GPU's stash instead of its own hidden
    activations: for rows of 1e6 or 1e30, a pre-activation that cancels to
    near zero carries an absolute rounding of ~2^-16 sum_i |x_i w_i| from
    the forward, so sigma(z) there is the forward's conditioning, not the
    backward's; on the same stash the backward is checked on its own."""
    x, ws = _inputs(dims, m, seed, wide_rows=wide_rows)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    rng = np.random.default_rng(seed + 1)
    if dout_mode == "scalar":  # loss = out.mean(): 1/(M * OUT) everywhere, far below fp16's normal range
        c = np.float32(1.0 / (m * dims[-1]))
        dout_np = np.full((m, dims[-1]), c, np.float64)
        dout = torch.full((), float(c), dtype=torch.float32, device="cuda").expand(m, dims[-1])
    else:
        dn = rng.standard_normal((m, dims[-1])).astype(np.float32)
        dout_np = dn.astype(np.float64)
        dout = torch.from_numpy(dn).cuda()
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    dx = torch.empty_like(xd) if with_dx else None
    ops.bwd(xd, wd, hs, dout, dws, dx)
    torch.cuda.synchronize()
    if own_stash:
        ref_h = [h.cpu().numpy().astype(np.float64) for h in hs]
    else:
        _, ref_h = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    rdws, rdx = orc.backward(x, ws, ref_h, dout_np, dtype=np.float64, need_dx=with_dx)
    return dws, dx, rdws, rdx


@pytest.mark.parametrize("m", [4096, 131072])
@pytest.mark.parametrize("dout_mode", ["dense", "scalar"])
def test_fp32_backward_matches_oracle(m, dout_mode):
    dims = (128, 128, 128, 128)
    dws, dx, rdws, rdx = _train32(dims, m, seed=m + 7, dout_mode=dout_mode, with_dx=True)
    for i in range(3):
        _check_dw32(dws[i].cpu().numpy(), rdws[i], f"fp32 dW{i + 1} M={m} {dout_mode}")
    _check_rows(dx.cpu().numpy(), rdx, f"fp32 dx M={m} {dout_mode}")


@pytest.mark.parametrize("m", [4096, 131072])
def test_fp32_backward_keeps_the_fp32_range(m):
    # Rows with |x| up to 1e30 and down to 1e-12 through the training forward
    # and the backward (on the forward's own stash, see _train32); dL/dout =
    # 1/(M * OUT) (a mean over the batch: fp16 would flush it to a subnormal).
    dims = (128, 128, 128, 128)
    dws, dx, rdws, rdx = _train32(dims, m, seed=m + 9, dout_mode="scalar", with_dx=True, wide_rows=True,
                                  own_stash=True)
    for i in range(3):
        g = dws[i].cpu().numpy()
        assert np.all(np.isfinite(g)), f"dW{i + 1} not finite"
        _check_dw32(g, rdws[i], f"fp32 range dW{i + 1} M={m}")
    _check_rows(dx.cpu().numpy(), rdx, f"fp32 range dx M={m}")


@pytest.mark.parametrize("dims,m", [((64, 96, 48, 16), 3001), ((48, 128, 32), 1000), ((128,) * 6, 4096),
                                    ((32, 64, 64, 16), 20000)])
def test_fp32_backward_runtime_widths(dims, m):
    dws, dx, rdws, rdx = _train32(dims, m, seed=m, dout_mode="dense", with_dx=True)
    for i in range(len(dims) - 1):
        _check_dw32(dws[i].cpu().numpy(), rdws[i], f"fp32 {dims} dW{i + 1}")
    _check_rows(dx.cpu().numpy(), rdx, f"fp32 {dims} dx")


def test_fp32_backward_support():
    assert ops.bwd_supported([128, 128, 128, 128])
    # fp32 widths stop at 128; mlpmk_bwd (no workspace) refuses fp32 tensors
    x = torch.zeros((64, 128), device="cuda")
    ws = [torch.zeros((128, 256), device="cuda"), torch.zeros((256, 128), device="cuda")]
    _, hs = ops.fwd(x.half(), [w.half() for w in ws], stash=True)
    dws = [torch.zeros(w.shape, device="cuda") for w in ws]
    with pytest.raises(ops.MlpmkError, match="UNSUPPORTED_SHAPE"):
        ops.bwd(x, ws, hs, torch.ones((64, 128), device="cuda"), dws)


# ---------------------------------------------------------------------------
# The drop-in modules with fp32 parameters and fp32 x outside autocast: fp32
# kernels, fp32 out, fp32 gradients (the reference's INPUT_DTYPE modules).
# ---------------------------------------------------------------------------

def _torch64(x, ws, wn_v=None, wn_g=None, dims=None):
    """float64 CPU autograd of the same network (optionally through weight
    norm): out, dx, parameter gradients for loss = out.sum()."""
    import torch.nn.functional as F
    xd = x.detach().cpu().double().requires_grad_(True)
    if wn_v is not None:
        v = wn_v.detach().cpu().double().requires_grad_(True)
        g = wn_g.detach().cpu().double().requires_grad_(True)
        ws64, vo, go = [], 0, 0
        for i in range(len(dims) - 1):
            k, n = dims[i], dims[i + 1]
            ws64.append(torch._weight_norm(v[vo:vo + k * n].view(k, n), g[go:go + n].view(1, n), dim=1))
            vo += k * n
            go += n
        params = [v, g]
    else:
        params = [w.detach().cpu().double().requires_grad_(True) for w in ws]
        ws64 = params
    a = xd
    for i, w in enumerate(ws64):
        a = a @ w
        if i < len(ws64) - 1:
            a = F.softplus(a)
    a.sum().backward()
    return a.detach().numpy(), xd.grad.numpy(), [p.grad.numpy() for p in params]


def _module_step(m, wn, big_rows, H=128, n_layers=3):
    import fused_mlp

    torch.manual_seed(11)
    model = (fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus)(H=H, n_layers=n_layers).cuda()
    x = torch.randn(m, 128, device="cuda")
    if big_rows:
        x[::5] *= 1e5  # rows past fp16's 65,504
    x.requires_grad_(True)
    out = model(x)
    assert out.dtype == torch.float32
    out.sum().backward()
    if wn:
        ref_out, ref_dx, ref_g = _torch64(x, None, model.v_all, model.g_all, model.dims)
        grads = [model.v_all.grad, model.g_all.grad]
    else:
        ref_out, ref_dx, ref_g = _torch64(x, list(model.weights))
        grads = [w.grad for w in model.weights]
    for gr in grads:
        assert gr.dtype == torch.float32 and bool(torch.isfinite(gr).all())
    return out, x.grad, grads, ref_out, ref_dx, ref_g


@pytest.mark.parametrize("m", [4096, 131072])
@pytest.mark.parametrize("wn", [False, True])
def test_fp32_modules_train_in_fp32(m, wn):
    out, gx, grads, ref_out, ref_dx, ref_g = _module_step(m, wn, big_rows=False)
    _check_rows(out.detach().cpu().numpy(), ref_out, f"module out M={m} wn={wn}")
    _check_rows(gx.cpu().numpy(), ref_dx, f"module dx M={m} wn={wn}")
    for i, (gr, rg) in enumerate(zip(grads, ref_g)):
        _check_dw32(gr.cpu().numpy().reshape(rg.shape), rg, f"module grad {i} M={m} wn={wn}")


@pytest.mark.parametrize("wn", [False, True])
def test_fp32_modules_with_rows_past_fp16_range(wn):
    # Every 5th row scaled by 1e5.  The outputs keep the row-scale bound.
    # The gradients of those rows depend on sigma(z) of pre-activations that
    # cancel to near zero, which the forward's operand rounding moves by
    # ~2^-16 sum_i |x_i w_i| (see _train32): there the gradients are finite
    # and the weight gradients within 5e-3 relative Frobenius (measured:
    # 3.5e-5 .. 6.8e-4); the other rows' dx keeps TOL.
    m = 4096
    out, gx, grads, ref_out, ref_dx, ref_g = _module_step(m, wn, big_rows=True)
    _check_rows(out.detach().cpu().numpy(), ref_out, f"module out wn={wn}")
    gx = gx.cpu().numpy()
    assert np.all(np.isfinite(gx))
    keep = np.ones(m, bool)
    keep[::5] = False
    _check_rows(gx[keep], ref_dx[keep], f"module dx wn={wn}")
    for i, (gr, rg) in enumerate(zip(grads, ref_g)):
        g = gr.cpu().numpy().reshape(rg.shape).astype(np.float64)
        frob = np.linalg.norm(g - rg) / np.linalg.norm(rg)
        assert frob < 5e-3, f"module grad {i} wn={wn}: rel frob {frob:.3g}"


# ---------------------------------------------------------------------------
# fp32 networks wider than 128: no fused fp32 kernel takes them, so they run
# layer by layer (mlpmk.fallback.fwd: fp32 library GEMMs and the library's
# fp32 softplus kernel, mlpmk_softplus_f32) and train through the fallback
# backward with every GEMM in fp32 -- fp32 in, fp32 out, fp32's range, as the
# reference's INPUT_DTYPE = fp32 kernels take any width (mlp_fused.md:159-166).
# ---------------------------------------------------------------------------

def test_softplus_f32_kernel_matches_torch_softplus():
    import torch.nn.functional as F
    from mlpmk import fallback

    edge = [-np.inf, -1000.0, -104.0, -88.0, -50.0, -20.0, -17.0, -10.0, -1e-3, -0.0, 0.0, 1e-3, 1.0, 10.0,
            19.99, 20.0, 20.01, 88.0, 1000.0, np.inf, np.nan]
    rng = np.random.default_rng(5)
    z = np.concatenate([np.array(edge, np.float32), (rng.standard_normal(10001) * 30).astype(np.float32)])
    zd = torch.from_numpy(z).cuda()
    got = fallback.softplus_f32(zd).cpu().numpy().astype(np.float64)
    ref = F.softplus(torch.from_numpy(z).double()).numpy()  # beta 1, threshold 20, as kernel.py:168-171
    assert np.isnan(got[20]) and got[0] == 0.0 and got[19] == np.inf
    fin = np.isfinite(ref)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=1e-6, atol=1e-37)
    assert np.all(got[fin] >= 0.0)
    # in place, and a length that leaves a tail past the 4-element steps
    zin = zd[:10003].clone()
    fallback.softplus_f32(zin, out=zin)
    np.testing.assert_array_equal(zin.cpu().numpy(), got[:10003].astype(np.float32))


@pytest.mark.parametrize("wn", [False, True])
@pytest.mark.parametrize("H,n_layers,m", [(256, 3, 4096), (192, 5, 2000), (320, 3, 1500)])
def test_fp32_modules_wider_than_128_train_in_fp32(wn, H, n_layers, m):
    from mlpmk import ops as _o

    dims = [128] + [H] * (n_layers - 1) + [128]
    assert not _o.fwd_supported(dims, torch.float32) and _o.fwd_supported(dims, torch.float16) == (H <= 256)
    out, gx, grads, ref_out, ref_dx, ref_g = _module_step(m, wn, big_rows=False, H=H, n_layers=n_layers)
    _check_rows(out.detach().cpu().numpy(), ref_out, f"module out H={H} wn={wn}", tol=1e-5)
    _check_rows(gx.cpu().numpy(), ref_dx, f"module dx H={H} wn={wn}", tol=1e-5)
    for i, (gr, rg) in enumerate(zip(grads, ref_g)):
        g = gr.cpu().numpy().reshape(rg.shape).astype(np.float64)
        frob = np.linalg.norm(g - rg) / np.linalg.norm(rg)
        assert frob < 1e-4, f"module grad {i} H={H} wn={wn}: rel frob {frob:.3g}"


def test_fp32_module_wider_than_128_keeps_rows_past_fp16_range():
    # Rows scaled by 1e5 stay finite in fp32 (in fp16 they would overflow).
    out, gx, grads, ref_out, ref_dx, ref_g = _module_step(4096, False, big_rows=True, H=256)
    assert float(out.detach().abs().max()) > 65504.0
    _check_rows(out.detach().cpu().numpy(), ref_out, "module out, rows past fp16 range", tol=1e-5)
    assert np.all(np.isfinite(gx.cpu().numpy()))
    for i, (gr, rg) in enumerate(zip(grads, ref_g)):
        g = gr.cpu().numpy().reshape(rg.shape).astype(np.float64)
        frob = np.linalg.norm(g - rg) / np.linalg.norm(rg)
        assert frob < 1e-4, f"module grad {i}: rel frob {frob:.3g}"


def test_fp32_launcher_wider_than_128_matches_model():
    rng = np.random.default_rng(9)
    dims = (128, 256, 256, 128)
    x = torch.from_numpy(rng.standard_normal((3000, 128)).astype(np.float32)).cuda()
    ws = [torch.from_numpy((rng.standard_normal((dims[i], dims[i + 1])) / np.sqrt(dims[i])).astype(np.float32)).cuda()
          for i in range(3)]
    out = kernel._fused_mlp_fwd(x, *ws)
    assert out.dtype == torch.float32
    ref = orc.forward(x.cpu().numpy(), [w.cpu().numpy() for w in ws], dtype=np.float64)
    _check_rows(out.cpu().numpy(), ref, "launcher fp32 H=256", tol=1e-5)
    eager = kernel.Model()(x, *ws)
    _check_rows(out.cpu().numpy(), eager.double().cpu().numpy(), "launcher fp32 H=256 vs eager Model", tol=1e-5)


def test_float64_module_runs_in_fp32():
    # float64 parameters and x: the network runs in fp32 (the widest type the
    # library computes in) and autograd hands float64 gradients back.
    import fused_mlp

    torch.manual_seed(12)
    model = fused_mlp.FusedMLPSoftplus().cuda().double()
    x = torch.randn(2048, 128, device="cuda", dtype=torch.float64).requires_grad_(True)
    out = model(x)
    assert out.dtype == torch.float32
    out.sum().backward()
    assert x.grad.dtype == torch.float64 and all(w.grad.dtype == torch.float64 for w in model.weights)
    ref_out, ref_dx, ref_g = _torch64(x, list(model.weights))
    _check_rows(out.detach().cpu().numpy(), ref_out, "fp64 module out")
    _check_rows(x.grad.cpu().numpy(), ref_dx, "fp64 module dx")
    for i, (w, rg) in enumerate(zip(model.weights, ref_g)):
        _check_dw32(w.grad.cpu().numpy(), rg, f"fp64 module dW{i + 1}")
