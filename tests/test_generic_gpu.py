"""Runtime-width kernels on the GPU: networks outside the three compiled
shapes (2..5 layers; input and hidden widths multiples of 16 up to 128; any
output width up to 128) run the library's width-128 kernels with the true
widths as launch parameters.  Parity against the CPU oracle on the same seeded
inputs, with the tolerances of test_fwd_gpu.py (outputs) and test_bwd_gpu.py
(gradients).  The reference's kernel takes any tile-multiple K1, N1, N2 and
masks N3 (/root/reference/kernel.py:60-63,86-87,121-123); its training
modules take D, H and out_features (/root/reference/README.md:62,68).
"""
import math

import numpy as np
import pytest
import torch

from oracle import mlp_oracle as orc
from mlpmk import ops
from test_bwd_gpu import check_dw

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-2

SHAPES = [
    (64, 64, 64, 64),
    (32, 128, 3),
    (16, 48, 80, 112, 7),
    (128, 96, 96, 96, 96, 40),
    (64, 128, 128, 1),
    (112, 32, 16),
    (128, 128, 128, 128, 128),
]


def _dev(x, ws):
    return torch.from_numpy(x).cuda(), [torch.from_numpy(w).cuda() for w in ws]


def _check(out, ref, what):
    ok, err, excess = orc.allclose_report(out, ref, ATOL, RTOL)
    assert ok, f"{what}: max|err|={err:.4g}, worst excess {excess:.4g}"


@pytest.mark.parametrize("dims", SHAPES)
@pytest.mark.parametrize("m", [1, 100, 5000, 70000])
def test_generic_forward_matches_oracle(dims, m):
    assert ops.fwd_supported(list(dims))
    x, ws = orc.make_inputs(dims, m, seed=m % 97)
    xd, wd = _dev(x, ws)
    out = ops.fwd(xd, wd)
    assert out.shape == (m, dims[-1])
    _check(out.float().cpu().numpy(), orc.forward(x, ws), f"{dims} M={m}")


@pytest.mark.parametrize("dims", [(64, 64, 64, 64), (32, 128, 3), (128, 96, 96, 96, 96, 40)])
def test_generic_stash_and_bit_identity(dims):
    m = 3000
    x, ws = orc.make_inputs(dims, m, seed=5)
    xd, wd = _dev(x, ws)
    out, hs = ops.fwd(xd, wd, stash=True)
    ref, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    _check(out.float().cpu().numpy(), ref, f"{dims} stash-mode out")
    for i, (h, rh) in enumerate(zip(hs, ref_h)):
        assert h.shape == (m, dims[i + 1])
        ok, err, _ = orc.allclose_report(h.cpu().numpy(), rh, 2e-3, 2e-3)
        assert ok, f"{dims} h{i + 1}: {err}"
    assert torch.equal(out, ops.fwd(xd, wd))  # inference and training forward agree bit for bit


@pytest.mark.parametrize("dims", [(64, 64, 64, 64), (16, 48, 80, 112, 7)])
def test_generic_launch_shapes_agree(dims):
    # 4-wave workgroups at M = 4096, 8-wave ones at M = 300000: same bits.
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn((300000, dims[0]), generator=g, device="cuda").half()
    ws = [(torch.randn((dims[i], dims[i + 1]), generator=g, device="cuda") / dims[i] ** 0.5).half()
          for i in range(len(dims) - 1)]
    big = ops.fwd(x, ws)
    small = ops.fwd(x[:4096].contiguous(), ws)
    assert torch.equal(big[:4096], small)
    xs = x[-200:].cpu().numpy()
    _check(big[-200:].float().cpu().numpy(), orc.forward(xs, [w.cpu().numpy() for w in ws]), f"{dims} tail")


@pytest.mark.parametrize("dims", [(64, 64, 64, 64), (32, 128, 3), (16, 48, 80, 112, 7),
                                  (128, 96, 96, 96, 96, 40), (112, 32, 16)])
@pytest.mark.parametrize("mode", ["dense", "ones"])
@pytest.mark.parametrize("with_dx", [False, True])
def test_generic_backward_matches_oracle(dims, mode, with_dx):
    m = 20000  # grids of 64+ workgroups: the partial-sum path
    x, ws = orc.make_inputs(dims, m, seed=7)
    xd, wd = _dev(x, ws)
    out, hs = ops.fwd(xd, wd, stash=True)
    if mode == "ones":
        dout_np = np.ones((m, dims[-1]), np.float16)
        dout = torch.ones((1, dims[-1]), dtype=torch.float16, device="cuda").expand(m, dims[-1])
    else:
        dout_np = np.random.default_rng(9).standard_normal((m, dims[-1])).astype(np.float16)
        dout = torch.from_numpy(dout_np).cuda()
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    dx = torch.empty_like(xd) if with_dx else None
    ops.bwd(xd, wd, hs, dout, dws, dx)
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, rdx = orc.backward(x, ws, ref_h, dout_np.astype(np.float32), need_dx=with_dx)
    for i in range(len(dws)):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"{dims} dW{i + 1}")
    if with_dx:
        _check(dx.float().cpu().numpy(), rdx, f"{dims} dx")


@pytest.mark.parametrize("dims,m", [((32, 128, 3), 1000), ((64, 64, 64, 64), 1)])
def test_generic_backward_small_grids_use_atomics(dims, m):
    # Below 64 workgroups the partials go to dW with fp32 atomics.
    x, ws = orc.make_inputs(dims, m, seed=11)
    xd, wd = _dev(x, ws)
    _, hs = ops.fwd(xd, wd, stash=True)
    dout_np = np.random.default_rng(3).standard_normal((m, dims[-1])).astype(np.float16)
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    ops.bwd(xd, wd, hs, torch.from_numpy(dout_np).cuda(), dws, workspace=False)
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, _ = orc.backward(x, ws, ref_h, dout_np.astype(np.float32), need_dx=False)
    for i in range(len(dws)):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"{dims} dW{i + 1}")


@pytest.mark.parametrize("D,H,OUT,L", [(64, 96, 3, 3), (32, 64, 5, 4), (48, 128, 16, 5)])
def test_generic_modules_train(D, H, OUT, L):
    import fused_mlp

    torch.manual_seed(0)
    for wn in (False, True):
        cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
        model = cls(D=D, H=H, out_features=OUT, n_layers=L).cuda()
        x = torch.randn(3000, D, device="cuda").half()
        out = model(x)
        assert out.shape == (3000, OUT)
        (out.float() * torch.linspace(-1, 1, OUT, device="cuda")).sum().backward()
        # torch float64 autograd of the same network on the CPU
        xr = x.double().cpu()
        params = [p.detach().double().cpu().requires_grad_(True) for p in model.parameters()]
        if wn:
            v_all, g_all = params
            dims = model.dims
            ws, vo, go = [], 0, 0
            for i in range(L):
                v = v_all[vo:vo + dims[i] * dims[i + 1]].reshape(dims[i], dims[i + 1])
                g = g_all[go:go + dims[i + 1]]
                ws.append((v * (g / v.norm(dim=0))).half().double())
                vo += dims[i] * dims[i + 1]
                go += dims[i + 1]
        else:
            ws = [p.half().double() for p in params]
        a = xr
        for i, w in enumerate(ws):
            a = a @ w
            if i < L - 1:
                a = torch.nn.functional.softplus(a).half().double()
        (a * torch.linspace(-1, 1, OUT, dtype=torch.float64)).sum().backward()
        ok, err, _ = orc.allclose_report(out.detach().float().cpu().numpy(), a.detach().numpy(), 1e-2, 1e-2)
        assert ok, f"{cls.__name__} {D, H, OUT, L} out: {err}"
        for p, r in zip(model.parameters(), params):
            check_dw(p.grad.cpu().numpy(), r.grad.numpy(), f"{cls.__name__} {D, H, OUT, L} grad")
        assert math.isfinite(float(out.detach().float().abs().max()))
