"""Pins the CPU oracle (oracle/mlp_oracle.py) before it is trusted as the
checker of the HIP kernels.

Each function is checked against something other than its own formula:
library routines (torch CPU float64: F.softplus, matmul, autograd,
torch._weight_norm), pure-Python math on the threshold edges, closed forms,
finite differences, and the committed golden fixtures (written by torch, not
by the oracle).  Planted mistakes -- the "branchless softplus" of
/root/reference/ablation_report.md:75-79, a transposed weight in the data
gradient, a dropped activation derivative, a weight norm over the wrong axis --
must each fail one of these checks.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mlp_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
EDGES = np.array([-200, -100, -30, -20.01, -20, -5, -1, -1e-3, 0, 1e-3, 0.5, 1, 5, 15, 19.99, 20, 20.01, 25, 60, 88, 1000],
                 dtype=np.float64)


def torch_forward(x, ws):
    a = torch.from_numpy(np.asarray(x, np.float64))
    for i, w in enumerate(ws):
        a = a @ torch.from_numpy(np.asarray(w, np.float64))
        if i < len(ws) - 1:
            a = F.softplus(a)  # beta=1, threshold=20, as kernel.py:108
    return a.numpy()


# ---------------------------------------------------------------- softplus --
def test_softplus_matches_torch_and_python_math_on_edges():
    got = orc.softplus(EDGES, np.float64)
    ref_t = F.softplus(torch.from_numpy(EDGES)).numpy()
    ref_py = np.array([z if z > 20 else math.log1p(math.exp(z)) for z in EDGES])
    np.testing.assert_allclose(got, ref_t, rtol=1e-12, atol=0)
    np.testing.assert_allclose(got, ref_py, rtol=1e-12, atol=0)
    assert got[EDGES == 0][0] == pytest.approx(math.log(2.0), rel=1e-15)


def test_softplus_fp32_grid():
    z = np.linspace(-40, 40, 100001, dtype=np.float32)
    np.testing.assert_allclose(orc.softplus(z), F.softplus(torch.from_numpy(z)).numpy(), rtol=4e-7, atol=1e-30)  # 2 ulp: numpy vs torch libm


def test_planted_branchless_softplus_is_caught():
    # ablation_report.md:75-79: "x + log(1 + exp(-|x|))" failed correctness.
    def buggy(z, dtype=np.float32):
        z = np.asarray(z, dtype=dtype)
        return (z + np.log1p(np.exp(-np.abs(z)))).astype(dtype)

    ref = F.softplus(torch.from_numpy(EDGES)).numpy()
    assert not np.allclose(buggy(EDGES, np.float64), ref, rtol=1e-2, atol=1e-2)


def test_softplus_grad_identity():
    z = np.linspace(-30, 30, 2001)
    zt = torch.from_numpy(z).requires_grad_(True)
    F.softplus(zt).sum().backward()
    h = orc.softplus(z, np.float64)
    # Above the threshold torch differentiates the linear branch (exactly 1);
    # 1 - exp(-h) (mlp_fused.md:57) is 1 - e^-z there, off by at most 2.1e-9.
    np.testing.assert_allclose(orc.softplus_grad_from_h(h, np.float64), zt.grad.numpy(), rtol=1e-9, atol=2.1e-9)
    below = z <= 20
    np.testing.assert_allclose(orc.softplus_grad_from_h(h[below], np.float64), zt.grad.numpy()[below], rtol=1e-9, atol=1e-15)


# ----------------------------------------------------------------- forward --
@pytest.mark.parametrize("dims", [(128, 128, 128, 128), (128,) * 6, (32, 64, 64, 16), (7, 5, 9, 3)])
def test_forward_matches_torch_float64(dims):
    x, ws = orc.make_inputs(dims, 300, seed=4, x_dist="normal")
    got = orc.forward(x, ws, dtype=np.float64)
    np.testing.assert_allclose(got, torch_forward(x, ws), rtol=1e-10, atol=1e-12)
    got32 = orc.forward(x, ws)
    np.testing.assert_allclose(got32, torch_forward(x, ws), rtol=1e-4, atol=1e-5)


def test_forward_zero_first_layer_closed_form():
    x, ws = orc.make_inputs((128, 128, 128, 128), 64, seed=2)
    ws[0] = np.zeros_like(ws[0])
    out = orc.forward(x, ws, dtype=np.float64)
    w2, w3 = ws[1].astype(np.float64), ws[2].astype(np.float64)
    row = np.log1p(np.exp(math.log(2.0) * w2.sum(axis=0))) @ w3
    np.testing.assert_allclose(out, np.broadcast_to(row, out.shape), rtol=1e-12, atol=1e-12)


def test_forward_identity_chain_is_double_softplus():
    z = EDGES.astype(np.float32)
    x = np.zeros((4, 32), np.float32)
    x[:, : z.size] = z
    eye = np.eye(32, dtype=np.float32)
    out = orc.forward(x, [eye, eye, eye], dtype=np.float64)
    def py_sp(v):
        return v if v > 20 else math.log1p(math.exp(v))

    expect = [py_sp(py_sp(float(v))) for v in x[0]]
    np.testing.assert_allclose(out[0], expect, rtol=1e-12, atol=1e-300)


def test_forward_linear_in_last_layer_and_row_independent():
    x, ws = orc.make_inputs((32, 64, 64, 16), 200, seed=9, x_dist="uniform")
    base = orc.forward(x, ws, dtype=np.float64)
    scaled = orc.forward(x, ws[:-1] + [ws[-1].astype(np.float64) * -3.5], dtype=np.float64)
    np.testing.assert_allclose(scaled, -3.5 * base, rtol=1e-12, atol=1e-14)
    perm = np.random.default_rng(0).permutation(200)
    np.testing.assert_array_equal(orc.forward(x[perm], ws, dtype=np.float64), base[perm])


def test_round_hidden_variant_stays_within_fp16_error():
    x, ws = orc.make_inputs((128, 128, 128, 128), 512, seed=1)
    a = orc.forward(x, ws)
    b = orc.forward(x, ws, round_hidden=True)
    assert np.max(np.abs(a - b)) < 5e-3


def test_to_bf16_matches_torch_conversion():
    # Random values over many binades, exact ties (even and odd kept bit),
    # values past the largest bf16 (round to inf), subnormals, signed zeros,
    # infinities and NaN: torch's float32 -> bfloat16 conversion is the check.
    rng = np.random.default_rng(0)
    a = (rng.standard_normal(200000) * np.exp2(rng.integers(-140, 127, 200000))).astype(np.float32)
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000, 0x7F7FFFFF, 0x00008000, 0x00018000],
                    dtype=np.uint32).view(np.float32)
    edge = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 3.4e38, -3.4e38, 1e-45, 1.17549435e-38], np.float32)
    a = np.concatenate([a, ties, edge])
    ref = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    got = orc.to_bf16(a)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even (1) wins; 1 + 3*2^-8 rounds up to 1 + 2^-6.
    assert orc.to_bf16(np.float32(1 + 2.0 ** -8)) == 1.0
    assert orc.to_bf16(np.float32(1 + 3 * 2.0 ** -8)) == np.float32(1 + 2.0 ** -6)


def test_round_hidden_bf16_variant_stays_within_bf16_error():
    x, ws = orc.make_inputs((128, 128, 128, 128), 512, seed=1, elem="bf16")
    assert np.array_equal(orc.to_bf16(x), x) and all(np.array_equal(orc.to_bf16(w), w) for w in ws)
    a = orc.forward(x, ws)
    b = orc.forward(x, ws, round_hidden=True, elem="bf16")
    c = orc.forward(x, ws, round_hidden=True)
    # bf16 keeps 8 significant bits against fp16's 11: about 8x the fp16 error.
    assert np.max(np.abs(a - b)) < 4e-2
    assert np.max(np.abs(a - c)) < np.max(np.abs(a - b))


# ---------------------------------------------------------------- backward --
def torch_grads(x, ws, dout):
    xt = torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True)
    wt = [torch.from_numpy(np.asarray(w, np.float64)).requires_grad_(True) for w in ws]
    a = xt
    for i, w in enumerate(wt):
        a = a @ w
        if i < len(wt) - 1:
            a = F.softplus(a)
    (a * torch.from_numpy(np.asarray(dout, np.float64))).sum().backward()
    return [w.grad.numpy() for w in wt], xt.grad.numpy()


@pytest.mark.parametrize("dims", [(128, 128, 128, 128), (32, 64, 64, 16), (6, 5, 7, 4), (128,) * 6])
def test_backward_matches_torch_autograd(dims):
    x, ws = orc.make_inputs(dims, 96, seed=3)
    dout = np.random.default_rng(5).standard_normal((96, dims[-1]))
    out, hs = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    dws, dx = orc.backward(x, ws, hs, dout, dtype=np.float64)
    tdws, tdx = torch_grads(x, ws, dout)
    for a, b in zip(dws, tdws):
        np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dx, tdx, rtol=1e-9, atol=1e-11)


def test_backward_broadcast_dout_equals_ones():
    x, ws = orc.make_inputs((128, 128, 128, 128), 64, seed=6)
    _, hs = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    a, adx = orc.backward(x, ws, hs, np.ones(128), dtype=np.float64)
    b, bdx = orc.backward(x, ws, hs, np.ones((64, 128)), dtype=np.float64)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)
    np.testing.assert_array_equal(adx, bdx)


def test_backward_finite_differences():
    rng = np.random.default_rng(11)
    dims = (3, 4, 5, 2)
    x = rng.standard_normal((5, 3))
    ws = [rng.standard_normal((dims[i], dims[i + 1])) for i in range(3)]
    dout = rng.standard_normal((5, 2))

    def loss(ws_, x_):
        return float((orc.forward(x_, ws_, dtype=np.float64) * dout).sum())

    _, hs = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    dws, dx = orc.backward(x, ws, hs, dout, dtype=np.float64)
    eps = 1e-6
    for li in range(3):
        num = np.zeros_like(ws[li])
        for idx in np.ndindex(*ws[li].shape):
            wp = [w.copy() for w in ws]
            wm = [w.copy() for w in ws]
            wp[li][idx] += eps
            wm[li][idx] -= eps
            num[idx] = (loss(wp, x) - loss(wm, x)) / (2 * eps)
        np.testing.assert_allclose(dws[li], num, rtol=1e-6, atol=1e-8)
    num = np.zeros_like(x)
    for idx in np.ndindex(*x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += eps
        xm[idx] -= eps
        num[idx] = (loss(ws, xp) - loss(ws, xm)) / (2 * eps)
    np.testing.assert_allclose(dx, num, rtol=1e-6, atol=1e-8)


def test_planted_backward_bugs_are_caught(monkeypatch):
    dims = (6, 5, 7, 4)
    x, ws = orc.make_inputs(dims, 40, seed=8)
    dout = np.random.default_rng(1).standard_normal((40, 4))
    _, hs = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    tdws, _ = torch_grads(x, ws, dout)

    def close(dws):
        return all(np.allclose(a, b, rtol=1e-3, atol=1e-6) for a, b in zip(dws, tdws))

    assert close(orc.backward(x, ws, hs, dout, dtype=np.float64)[0])
    # dropped activation derivative
    monkeypatch.setattr(orc, "softplus_grad_from_h", lambda h, dtype=np.float32: np.ones_like(h))
    assert not close(orc.backward(x, ws, hs, dout, dtype=np.float64)[0])
    monkeypatch.undo()
    # derivative from z instead of h (1 - exp(-z))
    monkeypatch.setattr(orc, "softplus_grad_from_h", lambda h, dtype=np.float32: 1 - np.exp(-np.asarray(h) * 0.5))
    assert not close(orc.backward(x, ws, hs, dout, dtype=np.float64)[0])


def test_planted_transposed_weight_in_data_gradient_is_caught():
    # Square layers so that a data gradient through W instead of W^T still runs.
    dims = (6, 6, 6, 6)
    x, ws = orc.make_inputs(dims, 30, seed=5)
    dout = np.random.default_rng(2).standard_normal((30, 6))
    _, hs = orc.forward(x, ws, dtype=np.float64, return_hidden=True)
    tdws, tdx = torch_grads(x, ws, dout)
    good, gdx = orc.backward(x, ws, hs, dout, dtype=np.float64)
    assert all(np.allclose(a, b, rtol=1e-6, atol=1e-9) for a, b in zip(good, tdws))
    # dz_{l-1} = (dz_l W_l) * sigma instead of (dz_l W_l^T) * sigma: feed W^T
    bad_ws = [w.T.copy() for w in ws]
    bad, bdx = orc.backward(x, bad_ws, hs, dout, dtype=np.float64)
    assert not np.allclose(bad[0], tdws[0], rtol=1e-3, atol=1e-6)
    assert not np.allclose(bdx, tdx, rtol=1e-3, atol=1e-6)


# --------------------------------------------------------------- weight norm --
def test_wn_forward_matches_torch_weight_norm_and_invariants():
    vs, gs = orc.make_wn_params((128, 128, 128, 128))
    rng = np.random.default_rng(2)
    for v, g in zip(vs, gs):
        g = g * rng.uniform(0.5, 2.0, size=g.shape).astype(np.float32)
        w, inv = orc.wn_forward(v, g, dtype=np.float64)
        tw = torch._weight_norm(torch.from_numpy(v.astype(np.float64)), torch.from_numpy(g.astype(np.float64))[None, :], 1)
        np.testing.assert_allclose(w, tw.numpy(), rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(np.linalg.norm(w, axis=0), np.abs(g), rtol=1e-12)
        np.testing.assert_allclose(inv, 1 / np.linalg.norm(v.astype(np.float64), axis=0), rtol=1e-12)


def test_wn_backward_matches_torch_autograd_and_invariants():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((32, 16))
    g = rng.uniform(0.5, 2, 16)
    dw = rng.standard_normal((32, 16))
    vt = torch.from_numpy(v).requires_grad_(True)
    gt = torch.from_numpy(g).requires_grad_(True)
    (torch._weight_norm(vt, gt[None, :], 1) * torch.from_numpy(dw)).sum().backward()
    dv, dg = orc.wn_backward(dw, v, g, dtype=np.float64)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, gt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose((dv * v).sum(axis=0), 0, atol=1e-10)  # dv is orthogonal to v
    w, _ = orc.wn_forward(v, g, dtype=np.float64)
    np.testing.assert_allclose(dg * g, (dw * w).sum(axis=0), rtol=1e-10)


def test_planted_wrong_norm_axis_is_caught():
    rng = np.random.default_rng(4)
    v = rng.standard_normal((16, 8))
    g = np.ones(8)
    tw = torch._weight_norm(torch.from_numpy(v), torch.from_numpy(g)[None, :], 1).numpy()
    wrong = v / np.linalg.norm(v, axis=1, keepdims=True)
    assert not np.allclose(wrong, tw, rtol=1e-3)


# ------------------------------------------------------------ golden fixtures --
def _golden(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.fail(f"missing fixture {path}; run tests/golden/make_golden.py")
    return np.load(path, allow_pickle=False)


@pytest.mark.parametrize("name", ["fwd_3l128_m256.npz", "fwd_5l128_m64.npz", "fwd_narrow_m64.npz"])
def test_oracle_matches_golden_forward(name):
    z = _golden(name)
    nl = int(z["num_layers"])
    ws = [z[f"w{i + 1}"] for i in range(nl)]
    got = orc.forward(z["x"], ws)
    np.testing.assert_allclose(got, z["out"], rtol=1e-4, atol=1e-5)


def test_oracle_matches_golden_training():
    z = _golden("train_wn_3l128_m64.npz")
    vs = [z[f"v{i + 1}"] for i in range(3)]
    gs = [z[f"g{i + 1}"] for i in range(3)]
    ws = []
    for i in range(3):
        w, _ = orc.wn_forward(vs[i], gs[i])
        np.testing.assert_allclose(w, z[f"w{i + 1}"], rtol=1e-5, atol=1e-7)
        ws.append(w)
    out, hs = orc.forward(z["x"], ws, return_hidden=True)
    np.testing.assert_allclose(out, z["out"], rtol=1e-4, atol=1e-5)
    dws, dx = orc.backward(z["x"], ws, hs, z["dout"])
    for i in range(3):
        np.testing.assert_allclose(dws[i], z[f"dw{i + 1}"], rtol=1e-4, atol=1e-4)
        dv, dg = orc.wn_backward(dws[i], vs[i], gs[i])
        np.testing.assert_allclose(dv, z[f"dv{i + 1}"], rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(dg, z[f"dg{i + 1}"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(dx, z["dx"], rtol=1e-4, atol=1e-5)
