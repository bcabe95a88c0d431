"""Recomputing backward of the 3- and 5-layer 128-wide networks: the training
forward does not write the last hidden activation h_{L-1}, and the backward
recomputes it, softplus(h_{L-2} W_{L-2}), for every block of rows instead of
reading it from the stash -- the activation recomputation the reference lists
as future work (/root/reference/mlp_fused.md:451-452) -- with or without dx.
Parity against the CPU oracle with the weight-gradient tolerance of
test_bwd_gpu.py (dx at 1e-2 / 1e-2), and against the stashing backward on the
same inputs.
"""
import numpy as np
import pytest
import torch

from oracle import mlp_oracle as orc
from mlpmk import ops
from test_bwd_gpu import check_dw

pytestmark = pytest.mark.gpu

D3 = [128, 128, 128, 128]


def _train(x, ws, dout_mode, recompute, workspace=True, seed=0):
    m = x.shape[0]
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out, hs = ops.fwd(xd, wd, stash=True, recompute=recompute)
    if dout_mode == "ones":
        dout_np = np.ones((m, 128), np.float16)
        dout = torch.ones((1, 128), dtype=torch.float16, device="cuda").expand(m, 128)
    else:
        dout_np = np.random.default_rng(seed + 5).standard_normal((m, 128)).astype(np.float16)
        dout = torch.from_numpy(dout_np).cuda()
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    ops.bwd(xd, wd, hs, dout, dws, None, workspace=workspace)
    torch.cuda.synchronize()
    return out, hs, [d.cpu().numpy() for d in dws], dout_np


def test_support_and_stash_layout():
    assert ops.bwd_recompute_supported(D3)
    assert ops.bwd_recompute_supported([128] * 6)
    for dims in ([128] * 5, [32, 64, 64, 16], [64, 64, 64, 64], [128, 256, 256, 128]):
        assert not ops.bwd_recompute_supported(dims), dims
    x, ws = orc.make_inputs(D3, 3000, seed=1)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out_full, hs_full = ops.fwd(xd, wd, stash=True)
    out_rc, hs_rc = ops.fwd(xd, wd, stash=True, recompute=True)
    assert hs_rc[1] is None
    # Skipping h_2 changes nothing else the forward writes.
    assert torch.equal(out_full, out_rc) and torch.equal(hs_full[0], hs_rc[0])


@pytest.mark.parametrize("m", [100, 5000, 131072])
def test_forward_without_h2_writes_the_same_bits(m):
    # Every launch shape (split kernel, 4-, 8- and 12-wave persistent kernels).
    g = torch.Generator(device="cuda").manual_seed(m)
    x = torch.randn((m, 128), generator=g, device="cuda").half()
    wd = [(torch.randn((128, 128), generator=g, device="cuda") / 128 ** 0.5).half() for _ in range(3)]
    out_full, hs_full = ops.fwd(x, wd, stash=True)
    out_rc, hs_rc = ops.fwd(x, wd, stash=True, recompute=True)
    assert torch.equal(out_full, out_rc) and torch.equal(hs_full[0], hs_rc[0])


@pytest.mark.parametrize("m", [1, 100, 4096, 20000, 131072])
@pytest.mark.parametrize("dout_mode", ["ones", "dense"])
def test_recompute_backward_matches_oracle_and_stash(m, dout_mode):
    x, ws = orc.make_inputs(D3, m, seed=m % 89)
    _, _, dws_rc, dout_np = _train(x, ws, dout_mode, recompute=True, seed=m)
    _, _, dws_st, _ = _train(x, ws, dout_mode, recompute=False, seed=m)
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, _ = orc.backward(x, ws, ref_h, dout_np.astype(np.float32), need_dx=False)
    for i in range(3):
        check_dw(dws_rc[i], rdws[i], f"recompute dW{i + 1} M={m} {dout_mode}")
        # The recomputed h_2 differs from the stashed one by fp16 operand
        # rounding at most: far below the oracle tolerance.
        diff = np.linalg.norm(dws_rc[i] - dws_st[i]) / max(np.linalg.norm(dws_st[i]), 1e-30)
        assert diff < 2e-3, f"dW{i + 1} M={m}: recompute vs stash rel frob {diff:.3g}"


def test_recompute_backward_atomic_flush():
    # Below 64 workgroups the weight-gradient partials go to dW with atomics.
    x, ws = orc.make_inputs(D3, 1000, seed=3)
    _, _, dws, dout_np = _train(x, ws, "dense", recompute=True, workspace=False, seed=3)
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, _ = orc.backward(x, ws, ref_h, dout_np.astype(np.float32), need_dx=False)
    for i in range(3):
        check_dw(dws[i], rdws[i], f"dW{i + 1} atomic")


def _rel(a, b):
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_recompute_overflowing_exponent():
    # x scaled by 300: pre-activations of ~1e3, 2^u overflows and the
    # recomputed softplus takes u itself.  Ordinary rows (every 7th) share
    # the blocks.
    m = 8192
    x, ws = orc.make_inputs(D3, m, seed=21)
    x = (x.astype(np.float32) * 300.0).astype(np.float16)
    small = np.zeros(m, dtype=bool)
    small[::7] = True
    x[small] = (x[small].astype(np.float32) / 300.0).astype(np.float16)
    _, _, dws_st, _ = _train(x, ws, "ones", recompute=False)
    _, _, dws_rc, _ = _train(x, ws, "ones", recompute=True)
    for i in range(3):
        assert np.isfinite(dws_rc[i]).all()
        assert _rel(dws_rc[i], dws_st[i]) < 2e-3, f"dW{i + 1}: {_rel(dws_rc[i], dws_st[i]):.3g}"


def test_recompute_operands_beyond_fp16():
    # Rows 0, 8, .., 56 of x point along sign(W1[:, 0]) so that h_1[:, 0]
    # lands in [47000, 60000]: finite in fp16 (the backward's exchange tiles
    # hold a_1 in fp16), but its base-2 value h_1 log2 e is beyond fp16, so the
    # recompute of those waves halves its operands and doubles the products.
    m = 4096
    x, ws = orc.make_inputs(D3, m, seed=8)
    w0 = ws[0][:, 0].astype(np.float64)
    targets = np.linspace(47000.0, 60000.0, 8)
    for r, t in zip(range(0, 64, 8), targets):
        x[r] = (np.sign(w0) * (t / np.abs(w0).sum())).astype(np.float16)
    _, hs_st, dws_st, _ = _train(x, ws, "ones", recompute=False)
    h1max = float(hs_st[0].max())
    assert 45500.0 < h1max < 65504.0, h1max  # the case this test is for
    for i in range(3):
        assert np.isfinite(dws_st[i]).all()
    _, _, dws_rc, _ = _train(x, ws, "ones", recompute=True)
    for i in range(3):
        assert np.isfinite(dws_rc[i]).all()
        assert _rel(dws_rc[i], dws_st[i]) < 2e-3, f"dW{i + 1}: {_rel(dws_rc[i], dws_st[i]):.3g}"


def _train_dx(dims, x, ws, dout_np, recompute):
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out, hs = ops.fwd(xd, wd, stash=True, recompute=recompute)
    dout = torch.from_numpy(dout_np).cuda()
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    dx = torch.empty_like(xd)
    ops.bwd(xd, wd, hs, dout, dws, dx)
    torch.cuda.synchronize()
    return out, hs, [d.cpu().numpy() for d in dws], dx.float().cpu().numpy()


@pytest.mark.parametrize("dims", [D3, [128] * 6])
@pytest.mark.parametrize("m", [100, 4096, 65536])
def test_recompute_backward_with_dx(dims, m):
    x, ws = orc.make_inputs(dims, m, seed=m % 37)
    dout_np = np.random.default_rng(m).standard_normal((m, dims[-1])).astype(np.float16)
    out_rc, hs_rc, dws_rc, dx_rc = _train_dx(dims, x, ws, dout_np, recompute=True)
    out_st, hs_st, dws_st, dx_st = _train_dx(dims, x, ws, dout_np, recompute=False)
    assert hs_rc[-1] is None and torch.equal(out_rc, out_st)
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, rdx = orc.backward(x, ws, ref_h, dout_np.astype(np.float32), need_dx=True)
    for i in range(len(dims) - 1):
        check_dw(dws_rc[i], rdws[i], f"recompute dW{i + 1} M={m}")
        assert _rel(dws_rc[i], dws_st[i]) < 2e-3, f"dW{i + 1} M={m}: recompute vs stash"
    ok, err, _ = orc.allclose_report(dx_rc, rdx, 1e-2, 1e-2)
    assert ok, f"dx M={m}: {err}"
    assert _rel(dx_rc, dx_st) < 2e-3


@pytest.mark.parametrize("m", [100, 5000, 131072])
def test_five_layer_forward_without_h4_writes_the_same_bits(m):
    g = torch.Generator(device="cuda").manual_seed(m)
    x = torch.randn((m, 128), generator=g, device="cuda").half()
    wd = [(torch.randn((128, 128), generator=g, device="cuda") / 128 ** 0.5).half() for _ in range(5)]
    out_full, hs_full = ops.fwd(x, wd, stash=True)
    out_rc, hs_rc = ops.fwd(x, wd, stash=True, recompute=True)
    assert hs_rc[3] is None and torch.equal(out_full, out_rc)
    for a, b in zip(hs_full[:3], hs_rc[:3]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("m", [4096, 131072])
@pytest.mark.parametrize("dout_mode", ["ones", "dense"])
def test_five_layer_recompute_backward_matches_oracle_and_stash(m, dout_mode):
    dims = [128] * 6
    x, ws = orc.make_inputs(dims, m, seed=m % 53)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    if dout_mode == "ones":
        dout_np = np.ones((m, 128), np.float16)
        dout = torch.ones((1, 128), dtype=torch.float16, device="cuda").expand(m, 128)
    else:
        dout_np = np.random.default_rng(m + 1).standard_normal((m, 128)).astype(np.float16)
        dout = torch.from_numpy(dout_np).cuda()
    res = {}
    for rc in (True, False):
        _, hs = ops.fwd(xd, wd, stash=True, recompute=rc)
        dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(5)]
        ops.bwd(xd, wd, hs, dout, dws, None)
        res[rc] = [d.cpu().numpy() for d in dws]
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, _ = orc.backward(x, ws, ref_h, dout_np.astype(np.float32), need_dx=False)
    for i in range(5):
        check_dw(res[True][i], rdws[i], f"5L recompute dW{i + 1} M={m} {dout_mode}")
        assert _rel(res[True][i], res[False][i]) < 2e-3, f"5L dW{i + 1} M={m}: recompute vs stash"


@pytest.mark.parametrize("wn", [False, True])
def test_modules_recompute_policy(wn):
    # The drop-in modules take the recomputing backward under RECOMPUTE =
    # "always" (and under "auto" from RECOMPUTE_MIN_ROWS rows for 3 layers,
    # RECOMPUTE_MIN_ROWS_5L for 5); the gradients agree with the stashing
    # path.
    import fused_mlp
    from mlpmk import autograd as mag

    torch.manual_seed(0)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls().cuda()
    x = torch.randn(5000, 128, device="cuda").half()
    assert mag._use_recompute(tuple(model.dims), 1 << 20, False)
    assert mag._use_recompute(tuple(model.dims), 1 << 20, True)  # dx too
    assert not mag._use_recompute(tuple(model.dims), 1 << 17, False)
    assert mag._use_recompute((128,) * 6, 1 << 17, False)
    assert not mag._use_recompute((128,) * 6, 1 << 16, False)
    assert not mag._use_recompute((128,) * 5, 1 << 20, False)  # 4 layers: no recomputing kernel
    grads = {}
    policy = mag.RECOMPUTE
    try:
        for pol in ("never", "always"):
            mag.RECOMPUTE = pol
            for p in model.parameters():
                p.grad = None
            xg = x.clone().requires_grad_(True)
            model(xg).float().sum().backward()  # dx wanted too
            grads[pol] = [p.grad.detach().float().cpu().numpy() for p in model.parameters()]
            grads[pol].append(xg.grad.float().cpu().numpy())
    finally:
        mag.RECOMPUTE = policy
    for a, b in zip(grads["always"], grads["never"]):
        assert _rel(a, b) < 2e-3


def test_five_layer_module_recompute_policy():
    import fused_mlp5
    from mlpmk import autograd as mag

    torch.manual_seed(1)
    model = fused_mlp5.FusedMLP5Softplus().cuda().half()
    x = torch.randn(4096, 128, device="cuda").half()
    grads = {}
    policy = mag.RECOMPUTE
    try:
        for pol in ("never", "always"):
            mag.RECOMPUTE = pol
            for p in model.parameters():
                p.grad = None
            xg = x.clone().requires_grad_(True)
            model(xg).float().sum().backward()
            grads[pol] = [p.grad.detach().float().cpu().numpy() for p in model.parameters()]
            grads[pol].append(xg.grad.float().cpu().numpy())
    finally:
        mag.RECOMPUTE = policy
    for a, b in zip(grads["always"], grads["never"]):
        assert _rel(a, b) < 2e-3
