"""Drop-in training modules and weight-norm kernels on the GPU.

* ``mlpmk_wn_fwd`` / ``mlpmk_wn_bwd`` (one launch each, all layers) against the
  CPU oracle, which tests/test_oracle.py pins to torch._weight_norm and autograd.
* ``fused_mlp.FusedMLPSoftplus`` / ``FusedMLPSoftplusWN`` (README.md:58-70
  usage: ``.cuda().half()``, ``out = model(x)``, ``out.sum().backward()``)
  against torch CPU float64 autograd of the same math on the same parameters.
* The committed golden training fixture (torch float64, 3L + weight norm,
  M = 64) through the WN module.

Tolerances: fp16 outputs atol = rtol = 1e-2; fp32 gradients per entry
|got - ref| <= 2e-2 |ref| + 2e-3 max|ref| and relative Frobenius < 1e-2
(the north_star's rtol 2e-2 with an atol scaled by the gradient's magnitude,
needed where entries cancel to near zero).
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fused_mlp
from oracle import mlp_oracle as orc
from mlpmk import ops

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def check_grad(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    bound = 2e-2 * np.abs(ref) + 2e-3 * scale
    worst = np.max(np.abs(got - ref) - bound)
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < 1e-2, f"{what}: worst excess {worst:.3g} (scale {scale:.3g}), rel frob {frob:.3g}"


def torch_ref(x16, ws16, dout=None):
    """float64 CPU autograd of the eager math (kernel.py:168-171) on the same
    fp16 values; returns out, grads of x and of every weight."""
    x = x16.detach().cpu().double().requires_grad_(True)
    ws = [w.detach().cpu().double().requires_grad_(True) for w in ws16]
    a = x
    for i, w in enumerate(ws):
        a = a @ w
        if i < len(ws) - 1:
            a = F.softplus(a)
    (a.sum() if dout is None else (a * dout.cpu().double()).sum()).backward()
    return a.detach().numpy(), x.grad.numpy(), [w.grad.numpy() for w in ws]


@pytest.mark.parametrize("dims,dtype", [((128, 128, 128, 128), torch.float32), ((128, 128, 128, 128), torch.float16),
                                        ((32, 64, 64, 16), torch.float32)])
def test_weight_norm_kernels(dims, dtype):
    vs, gs = orc.make_wn_params(dims, seed=4)
    rng = np.random.default_rng(8)
    gs = [g * rng.uniform(0.5, 2.0, g.shape).astype(np.float32) for g in gs]
    v_all = torch.from_numpy(np.concatenate([v.reshape(-1) for v in vs])).to("cuda", dtype)
    g_all = torch.from_numpy(np.concatenate(gs)).to("cuda", dtype)
    nw = v_all.numel()
    w_all = torch.empty(nw, dtype=torch.float16, device="cuda")
    inv_all = torch.empty(g_all.numel(), dtype=torch.float32, device="cuda")
    ops.wn_fwd(list(dims), v_all, g_all, w_all, inv_all)
    dw_all = torch.from_numpy(rng.standard_normal(nw).astype(np.float32)).cuda()
    dv_all, dg_all = torch.empty_like(v_all), torch.empty_like(g_all)
    ops.wn_bwd(list(dims), dw_all, v_all, g_all, inv_all, dv_all, dg_all)
    torch.cuda.synchronize()
    vo = go = 0
    v_np = v_all.float().cpu().numpy()
    g_np = g_all.float().cpu().numpy()
    for i in range(len(dims) - 1):
        k, n = dims[i], dims[i + 1]
        v = v_np[vo:vo + k * n].reshape(k, n)
        g = g_np[go:go + n]
        w_ref, inv_ref = orc.wn_forward(v, g, dtype=np.float64)
        np.testing.assert_allclose(w_all[vo:vo + k * n].float().cpu().numpy().reshape(k, n), w_ref,
                                   rtol=1e-3, atol=1e-3 * np.abs(w_ref).max())
        np.testing.assert_allclose(inv_all[go:go + n].cpu().numpy(), inv_ref, rtol=1e-5)
        dv_ref, dg_ref = orc.wn_backward(dw_all[vo:vo + k * n].cpu().numpy().reshape(k, n), v, g, dtype=np.float64)
        tol = 2e-3 if dtype == torch.float16 else 1e-5
        np.testing.assert_allclose(dv_all[vo:vo + k * n].float().cpu().numpy().reshape(k, n), dv_ref,
                                   rtol=tol, atol=tol * np.abs(dv_ref).max())
        np.testing.assert_allclose(dg_all[go:go + n].float().cpu().numpy(), dg_ref, rtol=tol,
                                   atol=tol * np.abs(dg_ref).max())
        vo += k * n
        go += n


@pytest.mark.parametrize("dims,m", [((128, 128, 128), 4096), ((32, 64, 16), 1000)])
def test_fused_mlp_softplus_module(dims, m):
    D, H, OUT = dims
    torch.manual_seed(0)
    model = fused_mlp.FusedMLPSoftplus(D=D, H=H, out_features=OUT).cuda().half()
    x = torch.randn(m, D, device="cuda").half().requires_grad_(True)
    out = model(x)
    out.sum().backward()  # loss of the README quick start
    ref_out, ref_dx, ref_dws = torch_ref(x, list(model.weights))
    ok, err, _ = orc.allclose_report(out.detach().float().cpu().numpy(), ref_out, 1e-2, 1e-2)
    assert ok, f"out: {err}"
    for i, w in enumerate(model.weights):
        assert w.grad is not None and w.grad.dtype == torch.float16
        check_grad(w.grad.float().cpu().numpy(), ref_dws[i], f"dW{i + 1}")
    ok, err, _ = orc.allclose_report(x.grad.float().cpu().numpy(), ref_dx, 1e-2, 1e-2)
    assert ok, f"dx: {err}"


def test_module_inference_under_no_grad_and_dense_dout():
    torch.manual_seed(1)
    model = fused_mlp.FusedMLPSoftplus().cuda().half()
    x = torch.randn(2048, 128, device="cuda").half()
    with torch.no_grad():
        out0 = model(x)
    out = model(x)
    assert torch.equal(out0, out.detach())
    dout = torch.randn_like(out)
    out.backward(dout)
    _, _, ref_dws = torch_ref(x, list(model.weights), dout=dout)
    for i, w in enumerate(model.weights):
        check_grad(w.grad.float().cpu().numpy(), ref_dws[i], f"dW{i + 1} dense dout")


def test_module_under_autocast_with_fp32_parameters():
    # AMP: fp32 master weights, fp16 autocast casts to fp16; grads come back fp32.
    torch.manual_seed(2)
    model = fused_mlp.FusedMLPSoftplus().cuda()
    x = torch.randn(1024, 128, device="cuda")
    with torch.autocast("cuda", dtype=torch.float16):
        out = model(x)
        assert out.dtype == torch.float16
    out.float().sum().backward()
    ref_out, _, ref_dws = torch_ref(x.half(), [w.half() for w in model.weights])
    for i, w in enumerate(model.weights):
        assert w.grad.dtype == torch.float32
        check_grad(w.grad.cpu().numpy(), ref_dws[i], f"AMP dW{i + 1}")


class _RecordStash:
    """Wraps ops._fwd_raw (every forward launch of the package goes through
    it) and records whether each launch wrote a stash."""

    def __init__(self, monkeypatch):
        self.calls = []
        real = ops._fwd_raw

        def fwd_raw(dev, dims, code, x_ptr, w_ptrs, out_ptr, stash_ptrs, M):
            self.calls.append(stash_ptrs is not None)
            return real(dev, dims, code, x_ptr, w_ptrs, out_ptr, stash_ptrs, M)

        monkeypatch.setattr(ops, "_fwd_raw", fwd_raw)


@pytest.mark.parametrize("wn", [False, True])
@pytest.mark.parametrize("mode", ["no_grad", "inference_mode", "no_requires_grad"])
def test_inference_writes_no_stash(monkeypatch, mode, wn):
    # Module inference must launch the plain forward, not the training
    # forward with its fp32 stash (0.5-1 GiB at 1M rows): under no_grad the
    # parameters still require grad, so ctx.needs_input_grad inside
    # Function.forward cannot tell.
    torch.manual_seed(3)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls().cuda().half()
    x = torch.randn(4096, 128, device="cuda").half()
    ref = model(x).detach()  # training forward (parameters require grad)
    rec = _RecordStash(monkeypatch)
    if mode == "no_grad":
        with torch.no_grad():
            out = model(x)
    elif mode == "inference_mode":
        with torch.inference_mode():
            out = model(x)
    else:
        for p_ in model.parameters():
            p_.requires_grad_(False)
        out = model(x)
    assert rec.calls == [False], rec.calls
    assert not out.requires_grad
    assert torch.equal(out, ref)  # inference and training forwards agree bit for bit
    model.zero_grad()
    for p_ in model.parameters():
        p_.requires_grad_(True)
    rec.calls.clear()
    model(x).sum().backward()
    assert rec.calls == [True]


@pytest.mark.parametrize("wn", [False, True])
def test_module_under_bf16_autocast_runs_bf16_kernels(wn):
    # torch.autocast(dtype=bfloat16): the bf16 kernels, not fp16 ones.
    torch.manual_seed(4)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls().cuda()
    x = torch.randn(2048, 128, device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = model(x)
        assert out.dtype == torch.bfloat16
    out.float().sum().backward()
    if wn:
        ws = [w.detach() for w in _wn_weights(model)]
    else:
        ws = [w.detach() for w in model.weights]
    xb = x.to(torch.bfloat16).float().cpu().numpy()
    wb = [orc.to_bf16(w.float().cpu().numpy()) for w in ws]
    ref = orc.forward(xb, wb, round_hidden=True, elem="bf16")
    ok, err, _ = orc.allclose_report(out.detach().float().cpu().numpy(), ref, 3e-2, 3e-2)  # bf16 tolerance, test_bf16_gpu.py
    assert ok, f"bf16 autocast out: {err}"
    for p_ in model.parameters():
        assert p_.grad is not None and p_.grad.dtype == torch.float32 and torch.isfinite(p_.grad).all()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        assert model(x).dtype == torch.bfloat16


def _wn_weights(model):
    """W_l = g v / ||v|| of a weight-norm module, fp32."""
    ws = []
    for i in range(len(model.dims) - 1):
        v = model.v(i).float()
        ws.append(model.g(i).float() * v / v.norm(dim=0, keepdim=True))
    return ws


def _torch_wn_ref(x16, v_all, g_all, dims):
    x = x16.detach().cpu().double()
    v = v_all.detach().cpu().double().requires_grad_(True)
    g = g_all.detach().cpu().double().requires_grad_(True)
    a, vo, go = x, 0, 0
    for i in range(len(dims) - 1):
        k, n = dims[i], dims[i + 1]
        vi = v[vo:vo + k * n].view(k, n)
        gi = g[go:go + n]
        w = torch._weight_norm(vi, gi.view(1, n), dim=1)  # norm over `in`, one per output column
        a = a @ w
        if i < len(dims) - 2:
            a = F.softplus(a)
        vo += k * n
        go += n
    a.sum().backward()
    return a.detach().numpy(), v.grad.numpy(), g.grad.numpy()


@pytest.mark.parametrize("m", [4096, 16384])
def test_fused_mlp_softplus_wn_module(m):
    torch.manual_seed(3)
    model = fused_mlp.FusedMLPSoftplusWN().cuda()
    with torch.no_grad():
        model.g_all.mul_(torch.rand_like(model.g_all) + 0.5)
    x = torch.randn(m, 128, device="cuda").half()
    out = model(x)
    out.sum().backward()
    ref_out, ref_dv, ref_dg = _torch_wn_ref(x, model.v_all, model.g_all, model.dims)
    ok, err, _ = orc.allclose_report(out.detach().float().cpu().numpy(), ref_out, 1e-2, 1e-2)
    assert ok, f"out: {err}"
    nw = 0
    for i in range(3):
        k, n = model.dims[i], model.dims[i + 1]
        check_grad(model.v_all.grad[nw:nw + k * n].cpu().numpy(), ref_dv[nw:nw + k * n], f"dv{i + 1}")
        nw += k * n
    check_grad(model.g_all.grad.cpu().numpy(), ref_dg, "dg")


def test_wn_module_matches_committed_golden_training_step():
    z = np.load(os.path.join(GOLDEN, "train_wn_3l128_m64.npz"))
    model = fused_mlp.FusedMLPSoftplusWN().cuda()
    with torch.no_grad():
        model.v_all.copy_(torch.from_numpy(np.concatenate([z[f"v{i}"].reshape(-1) for i in (1, 2, 3)])))
        model.g_all.copy_(torch.from_numpy(np.concatenate([z[f"g{i}"] for i in (1, 2, 3)])))
    x = torch.from_numpy(z["x"]).cuda().requires_grad_(True)
    out = model(x)
    out.backward(torch.from_numpy(z["dout"]).cuda().half())
    ok, err, _ = orc.allclose_report(out.detach().float().cpu().numpy(), z["out"], 1e-2, 1e-2)
    assert ok, f"out: {err}"
    nw, ng = 0, 0
    for i in (1, 2, 3):
        k, n = z[f"v{i}"].shape
        check_grad(model.v_all.grad[nw:nw + k * n].cpu().numpy().reshape(k, n), z[f"dv{i}"], f"golden dv{i}")
        check_grad(model.g_all.grad[ng:ng + n].cpu().numpy(), z[f"dg{i}"], f"golden dg{i}")
        nw += k * n
        ng += n
    ok, err, _ = orc.allclose_report(x.grad.float().cpu().numpy(), z["dx"], 1e-2, 1e-2)
    assert ok, f"dx: {err}"


def test_five_layer_module_forward_and_backward():
    # The 5-layer backward runs as two launches (layers 4..3 as a segment
    # handing fp16 dz_2 to layers 2..0 through the workspace).
    import fused_mlp5

    torch.manual_seed(4)
    model = fused_mlp5.FusedMLP5Softplus().cuda().half()
    x = torch.randn(4096, 128, device="cuda").half().requires_grad_(True)
    with torch.no_grad():
        out = model(x)
    ref_out, ref_dx, ref_dws = torch_ref(x, list(model.weights))
    ok, err, _ = orc.allclose_report(out.float().cpu().numpy(), ref_out, 1e-2, 1e-2)
    assert ok, err
    model(x).sum().backward()
    for i, w in enumerate(model.weights):
        check_grad(w.grad.float().cpu().numpy(), ref_dws[i], f"dW{i + 1}")
    ok, err, _ = orc.allclose_report(x.grad.float().cpu().numpy(), ref_dx, 1e-2, 1e-2)
    assert ok, f"dx: {err}"


@pytest.mark.parametrize("m", [4096, 65536])
def test_five_layer_wn_module(m):
    import fused_mlp5

    torch.manual_seed(6)
    model = fused_mlp5.FusedMLP5SoftplusWN().cuda()
    with torch.no_grad():
        model.g_all.mul_(torch.rand_like(model.g_all) + 0.5)
    x = torch.randn(m, 128, device="cuda").half()
    out = model(x)
    out.sum().backward()
    ref_out, ref_dv, ref_dg = _torch_wn_ref(x, model.v_all, model.g_all, model.dims)
    ok, err, _ = orc.allclose_report(out.detach().float().cpu().numpy(), ref_out, 1e-2, 1e-2)
    assert ok, f"out: {err}"
    nw = 0
    for i in range(5):
        k, n = model.dims[i], model.dims[i + 1]
        check_grad(model.v_all.grad[nw:nw + k * n].cpu().numpy(), ref_dv[nw:nw + k * n], f"dv{i + 1}")
        nw += k * n
    check_grad(model.g_all.grad.cpu().numpy(), ref_dg, "dg")


@pytest.mark.parametrize("wn", [False, True])
def test_empty_batch_trains_to_zero_gradients(wn):
    # M = 0: the forward returns [0, OUT], and out.sum().backward() (whose
    # gradient is one element expanded over nothing) gives zero weight
    # gradients through the fused backward.
    torch.manual_seed(5)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls().cuda()
    x = torch.randn(0, 128, device="cuda").half()
    out = model(x)
    assert tuple(out.shape) == (0, 128) and out.dtype == torch.float16
    out.sum().backward()
    for p_ in model.parameters():
        assert p_.grad is not None and p_.grad.shape == p_.shape
        assert torch.count_nonzero(p_.grad) == 0
    with torch.no_grad():
        assert tuple(model(x).shape) == (0, 128)


@pytest.mark.parametrize("wn", [False, True])
def test_second_derivative_raises_instead_of_returning_zeros(wn):
    # The library's gradients are written through raw pointers and carry no
    # autograd graph, so a double backward would silently treat them as
    # constants where dL/dout itself depends on the inputs (loss = sum(out^2));
    # the backward is marked once-differentiable and raises instead.
    model = (fused_mlp.FusedMLPSoftplusWN() if wn else fused_mlp.FusedMLPSoftplus()).cuda()
    x = torch.randn(64, 128, device="cuda").half().requires_grad_(True)
    out = model(x)
    (gx,) = torch.autograd.grad((out.float() ** 2).sum(), x, create_graph=True)
    assert gx.shape == x.shape
    with pytest.raises(RuntimeError, match="differentiate twice"):
        gx.float().sum().backward()
