"""bf16 tensors on the GPU: the forward, training forward, backward (stashing
and recomputing) and weight norm with bf16 x, W, out, dout and dx -- the
reference's INPUT_DTYPE kernels (/root/reference/mlp_fused.md:159-166), which
cast every tile to the input dtype and accumulate in fp32.

Tolerances.  bf16 keeps 8 significant bits (2^-9 relative rounding) where
fp16 keeps 11.  Against the oracle with the reference's bf16 roundings (x, W
and every hidden activation rounded to bf16) the kernels differ by their own
bf16 roundings: hidden activations rounded in base-2 units, and W1 and WL
staged times log2 e and ln 2 -- each at most 2^-9 relative.  Simulated on the
CPU over 20,000 rows of the three compiled shapes these reach 1.8 %-2.0 % of
an output at worst, so outputs are checked at atol = rtol = 3e-2 (fp16:
1e-2).  Weight gradients: |err| <= 4e-2 |ref| + (L + 1) 1e-3 max|ref| for an
L-layer network (the data gradient is rounded to bf16 once per layer on its
way down) and a relative Frobenius error below 2e-2 (fp16: 2e-2, 2e-3,
1e-2).
"""
import numpy as np
import pytest
import torch

from oracle import mlp_oracle as orc
from mlpmk import ops

pytestmark = pytest.mark.gpu

TOL = 3e-2
BF = torch.bfloat16

D3 = (128, 128, 128, 128)
D5 = (128,) * 6
NARROW = (32, 64, 64, 16)


def _dev(x, ws):
    return torch.from_numpy(x).cuda().to(BF), [torch.from_numpy(w).cuda().to(BF) for w in ws]


def _check(out, ref, what, tol=TOL):
    ok, err, excess = orc.allclose_report(out, ref, tol, tol)
    assert ok, f"{what}: max|err|={err:.4g}, worst excess {excess:.4g}"


def check_dw_bf16(got, ref, what, n_layers=3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    worst = np.max(np.abs(got - ref) - (4e-2 * np.abs(ref) + (n_layers + 1) * 1e-3 * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < 2e-2, f"{what}: worst excess {worst:.3g} (scale {scale:.3g}), rel frob {frob:.3g}"
    return frob


def _ref_fwd(x, ws, **kw):
    return orc.forward(x, ws, round_hidden=True, elem="bf16", **kw)


@pytest.mark.parametrize("dims,xd", [(D3, "normal"), (D5, "normal"), (NARROW, "uniform"),
                                     ((64, 96, 96, 3), "normal"), ((16, 48, 80, 112, 7), "normal")])
@pytest.mark.parametrize("m", [1, 100, 5000, 70000])
def test_bf16_forward_matches_oracle(dims, xd, m):
    x, ws = orc.make_inputs(dims, m, seed=m % 91, x_dist=xd, elem="bf16")
    xd_, wd = _dev(x, ws)
    out = ops.fwd(xd_, wd)
    assert out.dtype == BF and out.shape == (m, dims[-1])
    _check(out.float().cpu().numpy(), _ref_fwd(x, ws), f"bf16 {dims} M={m}")


@pytest.mark.parametrize("dims", [D3, D5, NARROW])
def test_bf16_launch_shapes_and_stash_agree(dims):
    # Feature-split kernel (M = 4096), 4-, 8- and 12/16-wave persistent
    # kernels (up to 1M rows), inference and training forward: same bits.
    g = torch.Generator(device="cuda").manual_seed(5)
    m = 1 << 20
    x = torch.randn((m, dims[0]), generator=g, device="cuda").to(BF)
    ws = [(torch.randn((dims[i], dims[i + 1]), generator=g, device="cuda") / dims[i] ** 0.5).to(BF)
          for i in range(len(dims) - 1)]
    big = ops.fwd(x, ws)
    for sm in (4096, 40000, 300000):
        assert torch.equal(big[:sm], ops.fwd(x[:sm].contiguous(), ws)), sm
    out_s, hs = ops.fwd(x[:40000].contiguous(), ws, stash=True)
    assert torch.equal(out_s, big[:40000])
    xs = x[-300:].float().cpu().numpy()
    wn = [w.float().cpu().numpy() for w in ws]
    _check(big[-300:].float().cpu().numpy(), _ref_fwd(xs, wn), f"bf16 {dims} tail")
    _, ref_h = _ref_fwd(x[:40000].float().cpu().numpy(), wn, return_hidden=True)
    for i, (h, rh) in enumerate(zip(hs, ref_h)):
        ok, err, _ = orc.allclose_report(h.cpu().numpy(), rh, TOL, TOL)
        assert ok, f"bf16 {dims} stash h{i + 1}: {err}"


def test_bf16_large_activations_take_the_exact_path():
    # x scaled by 300: 2^u overflows in every block; every 7th row keeps its scale.
    m = 16384
    x, ws = orc.make_inputs(D3, m, seed=21, elem="bf16")
    x = orc.to_bf16(x * 300.0)
    small = np.zeros(m, dtype=bool)
    small[::7] = True
    x[small] = orc.to_bf16(x[small] / 300.0)
    xd, wd = _dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    ref = _ref_fwd(x, ws)
    assert np.isfinite(out).all()
    _check(out[small], ref[small], "bf16 ordinary rows in exact-path blocks")
    big_err = np.abs(out[~small] - ref[~small]).max()
    assert big_err <= 1e-2 * np.abs(ref[~small]).max()


def _train(dims, m, seed, dout_mode, with_dx, recompute=False, workspace=True):
    x, ws = orc.make_inputs(dims, m, seed=seed, elem="bf16")
    xd, wd = _dev(x, ws)
    out, hs = ops.fwd(xd, wd, stash=True, recompute=recompute)
    if dout_mode == "ones":
        dout_np = np.ones((m, dims[-1]), np.float32)
        dout = torch.ones((1, dims[-1]), dtype=BF, device="cuda").expand(m, dims[-1])
    else:
        dout_np = orc.to_bf16(np.random.default_rng(seed + 1).standard_normal((m, dims[-1])).astype(np.float32))
        dout = torch.from_numpy(dout_np).cuda().to(BF)
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    dx = torch.empty_like(xd) if with_dx else None
    ops.bwd(xd, wd, hs, dout, dws, dx, workspace=workspace)
    torch.cuda.synchronize()
    _, ref_h = _ref_fwd(x, ws, return_hidden=True)
    rdws, rdx = orc.backward(x, ws, ref_h, dout_np, need_dx=with_dx)
    return [d.cpu().numpy() for d in dws], dx, rdws, rdx


# Widths up to 128 take the two-pass backward at 300 rows and the one-pass
# megakernel above 16,384; 128-256-256-128 (streamed-weight forward) takes
# the two-pass form at every size.
@pytest.mark.parametrize("dims", [D3, D5, NARROW, (64, 96, 96, 3), (128, 256, 256, 128)])
@pytest.mark.parametrize("m,dout_mode", [(300, "dense"), (20000, "ones"), (131072, "dense")])
def test_bf16_backward_matches_oracle(dims, m, dout_mode):
    dws, dx, rdws, rdx = _train(dims, m, seed=m % 83, dout_mode=dout_mode, with_dx=True)
    for i in range(len(dws)):
        check_dw_bf16(dws[i], rdws[i], f"bf16 {dims} dW{i + 1} M={m}", len(dims) - 1)
    _check(dx.float().cpu().numpy(), rdx, f"bf16 {dims} dx M={m}")


def test_bf16_backward_atomic_flush_and_recompute():
    dws, _, rdws, _ = _train(D3, 1000, seed=4, dout_mode="dense", with_dx=False, workspace=False)
    for i in range(3):
        check_dw_bf16(dws[i], rdws[i], f"bf16 atomic dW{i + 1}")
    dws_rc, _, rdws, _ = _train(D3, 50000, seed=6, dout_mode="ones", with_dx=False, recompute=True)
    dws_st, _, _, _ = _train(D3, 50000, seed=6, dout_mode="ones", with_dx=False)
    for i in range(3):
        check_dw_bf16(dws_rc[i], rdws[i], f"bf16 recompute dW{i + 1}")
        rel = np.linalg.norm(dws_rc[i] - dws_st[i]) / np.linalg.norm(dws_st[i])
        assert rel < 5e-3, f"bf16 recompute vs stash dW{i + 1}: {rel:.3g}"


@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
def test_bf16_weight_norm(pdt):
    dims = D3
    vs, gs = orc.make_wn_params(dims, seed=3)
    gs = [g * np.linspace(0.5, 2.0, g.size, dtype=np.float32) for g in gs]
    if pdt == torch.bfloat16:
        vs = [orc.to_bf16(v) for v in vs]
        gs = [orc.to_bf16(g) for g in gs]
    v_all = torch.from_numpy(np.concatenate([v.reshape(-1) for v in vs])).cuda().to(pdt)
    g_all = torch.from_numpy(np.concatenate(gs)).cuda().to(pdt)
    nw = sum(dims[i] * dims[i + 1] for i in range(3))
    w_all = torch.empty(nw, dtype=BF, device="cuda")
    inv = torch.empty(sum(dims[1:]), dtype=torch.float32, device="cuda")
    ops.wn_fwd(dims, v_all, g_all, w_all, inv)
    off = 0
    for i in range(3):
        rw, rinv = orc.wn_forward(vs[i], gs[i])
        n = dims[i] * dims[i + 1]
        got = w_all[off:off + n].float().cpu().numpy().reshape(dims[i], dims[i + 1])
        assert np.array_equal(got, orc.to_bf16(rw)) or np.abs(got - rw).max() <= 2 ** -8 * np.abs(rw).max()
        off += n
    dw_all = torch.randn(nw, device="cuda")
    dv = torch.empty_like(v_all)
    dg = torch.empty_like(g_all)
    ops.wn_bwd(dims, dw_all, v_all, g_all, inv, dv, dg)
    dwn = dw_all.cpu().numpy()
    off = goff = 0
    for i in range(3):
        n = dims[i] * dims[i + 1]
        rdv, rdg = orc.wn_backward(dwn[off:off + n].reshape(dims[i], dims[i + 1]), vs[i], gs[i])
        tol = 1e-5 if pdt == torch.float32 else 1e-2
        gv = dv[off:off + n].float().cpu().numpy().reshape(dims[i], dims[i + 1])
        assert np.abs(gv - rdv).max() <= tol * np.abs(rdv).max() + 1e-6
        gg = dg[goff:goff + dims[i + 1]].float().cpu().numpy()
        assert np.abs(gg - rdg).max() <= tol * np.abs(rdg).max() + 1e-6
        off += n
        goff += dims[i + 1]


@pytest.mark.parametrize("wn", [False, True])
def test_bf16_modules_train(wn):
    # A bf16 x runs the bf16 kernels; gradients against float64 autograd of
    # the same network with bf16 roundings of x, W and the hidden activations.
    import fused_mlp

    torch.manual_seed(0)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls(D=64, H=128, out_features=10).cuda()
    x = torch.randn(6000, 64, device="cuda").to(BF)
    out = model(x)
    assert out.dtype == BF
    wts = torch.linspace(-1, 1, 10, device="cuda")
    (out.float() * wts).sum().backward()
    params = [p.detach().double().cpu().requires_grad_(True) for p in model.parameters()]
    dims = model.dims
    if wn:
        v_all, g_all = params
        ws, vo, go = [], 0, 0
        for i in range(3):
            v = v_all[vo:vo + dims[i] * dims[i + 1]].reshape(dims[i], dims[i + 1])
            gg = g_all[go:go + dims[i + 1]]
            ws.append(v * (gg / v.norm(dim=0)))
            vo += dims[i] * dims[i + 1]
            go += dims[i + 1]
    else:
        ws = list(params)
    bfr = lambda t: t + (t.to(torch.bfloat16).double() - t).detach()  # noqa: E731  (bf16 value, identity gradient)
    a = x.double().cpu()
    for i, w in enumerate(ws):
        a = a @ bfr(w)
        if i < 2:
            a = bfr(torch.nn.functional.softplus(a))
    (a * wts.double().cpu()).sum().backward()
    _check(out.detach().float().cpu().numpy(), a.detach().numpy(), f"{cls.__name__} bf16 out")
    for p, r in zip(model.parameters(), params):
        check_dw_bf16(p.grad.float().cpu().numpy(), r.grad.numpy(), f"{cls.__name__} bf16 grad")
