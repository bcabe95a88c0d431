"""The reference's large-M backward fallback (mlp_fused.md:114-146) as a
component: the ``mlpmk_sigmoid_h_mul`` HIP kernel against numpy, and the
interleaved GEMM + sigmoid_h_mul backward (``mlpmk.fallback.bwd``) against the
CPU oracle, against the fused backward megakernel, and through the drop-in
module with ``autograd.BACKWARD = "fallback"``.

Tolerances as for the fused backward: fp32 weight gradients per entry within
2e-2 |ref| + 2e-3 max|ref| and relative Frobenius 1e-2; dx at 1e-2 / 1e-2.
"""
import numpy as np
import pytest
import torch

import fused_mlp
from mlpmk import autograd as mag
from mlpmk import fallback, ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu


def check_grad(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    worst = np.max(np.abs(got - ref) - (2e-2 * np.abs(ref) + 2e-3 * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < 1e-2, f"{what}: worst excess {worst:.3g}, rel frob {frob:.3g}"


@pytest.mark.parametrize("n", [8, 1000, 4099, 1 << 20])
@pytest.mark.parametrize("dh_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_sigmoid_h_mul_kernel(n, dh_dtype):
    g = torch.Generator(device="cuda").manual_seed(n)
    # h >= 0 over the whole range: 0, saturated units (softplus(-20) ~ 2e-9), ~1, large, inf
    h = torch.rand(n, generator=g, device="cuda") * 30.0
    h[::7] = torch.exp(-torch.rand(n, generator=g, device="cuda")[::7] * 25.0)
    h[0] = 0.0
    if n > 5:
        h[5] = float("inf")
    dh = (torch.randn(n, generator=g, device="cuda") * 3.0).to(dh_dtype)
    dz32, dz16 = fallback.sigmoid_h_mul(h, dh, dz16_dtype=torch.float16)
    hn = h.cpu().double().numpy()
    ref = dh.float().cpu().double().numpy() * -np.expm1(-hn)
    got = dz32.cpu().double().numpy()
    err = np.abs(got - ref)
    assert np.all(err <= 1e-5 * np.abs(ref) + 1e-30), float((err / np.maximum(np.abs(ref), 1e-30)).max())
    assert torch.equal(dz16, dz32.half())


@pytest.mark.parametrize("dims,m", [((128, 128, 128, 128), 4096), ((128, 128, 128, 128), 131072),
                                    ((128,) * 6, 16384), ((32, 64, 64, 16), 4096)])
@pytest.mark.parametrize("dense", [False, True])
@pytest.mark.parametrize("with_dx", [False, True])
def test_fallback_backward_matches_oracle_and_fused(dims, m, dense, with_dx):
    x, ws = orc.make_inputs(dims, m, seed=3, x_dist="uniform" if dims[0] == 32 else "normal")
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    if dense:
        g = torch.Generator(device="cuda").manual_seed(9)
        dout = torch.randn((m, dims[-1]), generator=g, device="cuda").half()
    else:
        dout = torch.ones((1, dims[-1]), dtype=torch.float16, device="cuda").expand(m, dims[-1])
    L = len(dims) - 1
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(L)]
    dx = torch.empty_like(xd) if with_dx else None
    fallback.bwd(xd, wd, hs, dout, dws, dx)
    fdws = [torch.zeros_like(d) for d in dws]
    fdx = torch.empty_like(xd) if with_dx else None
    ops.bwd(xd, wd, hs, dout, fdws, fdx)
    rdws, rdx = orc.backward(x, ws, [h.cpu().numpy() for h in hs], dout.float().cpu().numpy(), need_dx=with_dx)
    for i in range(L):
        check_grad(dws[i].cpu().numpy(), rdws[i], f"fallback dW{i + 1}")
        check_grad(dws[i].cpu().numpy(), fdws[i].cpu().numpy(), f"fallback vs fused dW{i + 1}")
    if with_dx:
        ok, err, _ = orc.allclose_report(dx.float().cpu().numpy(), rdx, 1e-2, 1e-2)
        assert ok, f"fallback dx: {err}"


def test_module_trains_through_the_fallback(monkeypatch):
    torch.manual_seed(5)
    model = fused_mlp.FusedMLPSoftplusWN().cuda()
    x = torch.randn(8192, 128, device="cuda").half()
    model(x).sum().backward()
    ref = (model.v_all.grad.clone(), model.g_all.grad.clone())
    model.zero_grad()
    monkeypatch.setattr(mag, "BACKWARD", "fallback")
    model(x).sum().backward()
    check_grad(model.v_all.grad.cpu().numpy(), ref[0].cpu().numpy(), "dv fallback vs fused")
    check_grad(model.g_all.grad.cpu().numpy(), ref[1].cpu().numpy(), "dg fallback vs fused")
