"""Recomputing backward of the 3-layer 128-wide network: the training forward
writes only h_1, and the backward recomputes h_2 = softplus(h_1 W_2) for every
block of rows from h_1 and W_2 instead of reading a stashed h_2 -- the
activation recomputation the reference lists as future work
(/root/reference/mlp_fused.md:451-452).  Parity against the CPU oracle with the
weight-gradient tolerance of test_bwd_gpu.py, and against the stashing
backward on the same inputs.
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
    assert not ops.bwd_recompute_supported([128] * 6)
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


def test_recompute_rejects_dx():
    x = torch.randn((256, 128), device="cuda").half()
    wd = [(torch.randn((128, 128), device="cuda") / 128 ** 0.5).half() for _ in range(3)]
    _, hs = ops.fwd(x, wd, stash=True, recompute=True)
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    dout = torch.ones((256, 128), dtype=torch.float16, device="cuda")
    with pytest.raises(ops.MlpmkError, match="dx"):
        ops.bwd(x, wd, hs, dout, dws, torch.empty_like(x))


@pytest.mark.parametrize("wn", [False, True])
def test_modules_recompute_policy(wn):
    # The drop-in modules take the recomputing backward under RECOMPUTE =
    # "always" (and from RECOMPUTE_MIN_ROWS rows under "auto"); the gradients
    # agree with the stashing path, and an x that needs grad keeps the stash.
    import fused_mlp
    from mlpmk import autograd as mag

    torch.manual_seed(0)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls().cuda()
    x = torch.randn(5000, 128, device="cuda").half()
    assert mag._use_recompute(tuple(model.dims), 1 << 20, False)
    assert not mag._use_recompute(tuple(model.dims), 1 << 20, True)
    assert not mag._use_recompute((128,) * 6, 1 << 20, False)
    grads = {}
    policy = mag.RECOMPUTE
    try:
        for pol in ("never", "always"):
            mag.RECOMPUTE = pol
            for p in model.parameters():
                p.grad = None
            model(x).float().sum().backward()
            grads[pol] = [p.grad.detach().float().cpu().numpy() for p in model.parameters()]
        xg = x.clone().requires_grad_(True)
        model(xg).float().sum().backward()  # dx wanted: the stash path
        assert xg.grad is not None and torch.isfinite(xg.grad).all()
    finally:
        mag.RECOMPUTE = policy
    for a, b in zip(grads["always"], grads["never"]):
        assert _rel(a, b) < 2e-3
