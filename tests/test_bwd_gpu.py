"""Backward megakernel parity on the GPU: HIP path (through the C ABI) vs the
CPU oracle's closed-form backward on the same seeded inputs.

The GPU forward writes the fp32 activation stash; the oracle backward is fed
the oracle's own hidden activations (fp32, computed from fp16-rounded layer
inputs exactly as the megakernel does), so the check covers the stash too.

Tolerances: fp32 weight gradients within rtol 2e-2.
A pure relative test fails on entries that are near zero by cancellation, so
each entry must satisfy |got - ref| <= 2e-2 * |ref| + 2e-3 * max|ref| (the
atol scaled by the gradient's own magnitude), and the relative Frobenius
error must stay below 1e-2.  fp16 dx within atol = rtol = 1e-2.
"""
import numpy as np
import pytest
import torch

from oracle import mlp_oracle as orc
from mlpmk import ops

pytestmark = pytest.mark.gpu

D3 = (128, 128, 128, 128)
D5 = (128,) * 6
NARROW = (32, 64, 64, 16)


def check_dw(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    bound = 2e-2 * np.abs(ref) + 2e-3 * scale
    worst = np.max(np.abs(got - ref) - bound)
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < 1e-2, f"{what}: worst excess {worst:.3g} (scale {scale:.3g}), rel frob {frob:.3g}"
    return frob


def run_train(dims, m, seed, *, dout_mode="ones", with_dx=True, x_dist="normal", workspace=True):
    x, ws = orc.make_inputs(dims, m, seed=seed, x_dist=x_dist)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out, hs = ops.fwd(xd, wd, stash=True)
    rng = np.random.default_rng(seed + 17)
    if dout_mode == "ones":
        dout_np = np.ones((m, dims[-1]), np.float16)
        dout = torch.ones((1, dims[-1]), dtype=torch.float16, device="cuda").expand(m, dims[-1])
    elif dout_mode == "row":
        row = rng.standard_normal(dims[-1]).astype(np.float16)
        dout_np = np.broadcast_to(row, (m, dims[-1]))
        dout = torch.from_numpy(row).cuda().reshape(1, -1).expand(m, dims[-1])
    elif dout_mode == "scalar":  # one element expanded everywhere, as loss = out.sum() hands back
        dout_np = np.full((m, dims[-1]), 0.75, np.float16)
        dout = torch.full((), 0.75, dtype=torch.float16, device="cuda").expand(m, dims[-1])
    else:
        dout_np = rng.standard_normal((m, dims[-1])).astype(np.float16)
        dout = torch.from_numpy(dout_np).cuda()
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    dx = torch.empty_like(xd) if with_dx else None
    ops.bwd(xd, wd, hs, dout, dws, dx, workspace=workspace)
    torch.cuda.synchronize()
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, rdx = orc.backward(x, ws, ref_h, dout_np.astype(np.float32), need_dx=with_dx)
    return out, hs, dws, dx, rdws, rdx


@pytest.mark.parametrize("m", [64, 256, 4096, 16384, 65536])
def test_3l128_weight_and_data_gradients(m):
    # (65536 rows: two rounds per workgroup of the 8-wave kernel with dx.)
    _, _, dws, dx, rdws, rdx = run_train(D3, m, seed=m)
    for i in range(3):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1} M={m}")
    ok, err, excess = orc.allclose_report(dx.float().cpu().numpy(), rdx, 1e-2, 1e-2)
    assert ok, f"dx M={m}: max err {err:.3g}, excess {excess:.3g}"


@pytest.mark.parametrize("m", [64, 4096, 16384, 65536])
def test_5l128_weight_and_data_gradients(m):
    # Two launches: layers 4..3 as a segment (its layer-0 activation is the
    # stash h_3, its data gradient the fp16 dz_2 in the workspace), then
    # layers 2..0 with dz_2 as their output gradient.
    _, _, dws, dx, rdws, rdx = run_train(D5, m, seed=50 + m)
    for i in range(5):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1} M={m}")
    ok, err, excess = orc.allclose_report(dx.float().cpu().numpy(), rdx, 1e-2, 1e-2)
    assert ok, f"dx M={m}: max err {err:.3g}, excess {excess:.3g}"


@pytest.mark.parametrize("m", [1, 33, 1000, 4097])
def test_5l128_ragged_rows_without_dx(m):
    _, _, dws, dx, rdws, _ = run_train(D5, m, seed=7 * m + 2, dout_mode="full", with_dx=False)
    assert dx is None
    for i in range(5):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1} M={m}")


def test_5l128_without_workspace_is_rejected():
    x, ws = orc.make_inputs(D5, 256, seed=9)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    dout = torch.ones((256, 128), dtype=torch.float16, device="cuda")
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(5)]
    with pytest.raises(ops.MlpmkError, match="mlpmk_bwd_ws"):
        ops.bwd(xd, wd, hs, dout, dws, workspace=False)
    torch.cuda.synchronize()
    assert all(float(d.abs().max()) == 0.0 for d in dws)


@pytest.mark.parametrize("m", [1, 31, 33, 129, 1000, 4097])
def test_3l128_ragged_rows_without_dx(m):
    # Rows past M must contribute nothing (their loads read zeros).
    _, _, dws, dx, rdws, _ = run_train(D3, m, seed=3 * m + 1, dout_mode="full", with_dx=False)
    assert dx is None
    for i in range(3):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1} M={m}")


@pytest.mark.parametrize("mode", ["row", "full"])
def test_3l128_dout_layouts(mode):
    # Broadcast rows (stride 0, the expanded grad of loss = out.sum()) and a
    # dense dout give the same results as the oracle.
    _, _, dws, dx, rdws, rdx = run_train(D3, 3000, seed=11, dout_mode=mode)
    for i in range(3):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1} {mode}")
    ok, err, _ = orc.allclose_report(dx.float().cpu().numpy(), rdx, 1e-2, 1e-2)
    assert ok, err


def test_3l128_training_config_m131072():
    # Training config at its largest M: the full gradients against the oracle.
    _, _, dws, _, rdws, _ = run_train(D3, 131072, seed=5, with_dx=False)
    for i in range(3):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1} M=131072")


def test_weight_gradients_accumulate():
    # dw is accumulated into (+=): a second call on the same buffers doubles it.
    x, ws = orc.make_inputs(D3, 2048, seed=9)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    dout = torch.ones((1, 128), dtype=torch.float16, device="cuda").expand(2048, 128)
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    ops.bwd(xd, wd, hs, dout, dws)
    once = [d.clone() for d in dws]
    ops.bwd(xd, wd, hs, dout, dws)
    for a, b in zip(once, dws):
        torch.testing.assert_close(b, 2 * a, rtol=1e-5, atol=1e-5 * float(a.abs().max()))


@pytest.mark.parametrize("m", [64, 1000, 65536])
def test_narrow_gradients(m):
    _, _, dws, dx, rdws, rdx = run_train(NARROW, m, seed=m + 2, x_dist="uniform", dout_mode="full")
    for i in range(3):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"narrow dW{i + 1} M={m}")
    ok, err, _ = orc.allclose_report(dx.float().cpu().numpy(), rdx, 1e-2, 1e-2)
    assert ok, err


def test_zero_dout_gives_zero_gradients():
    x, ws = orc.make_inputs(D3, 512, seed=1)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    dout = torch.zeros((512, 128), dtype=torch.float16, device="cuda")
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    dx = torch.full_like(xd, 7.0)
    ops.bwd(xd, wd, hs, dout, dws, dx)
    assert all(float(d.abs().max()) == 0.0 for d in dws)
    assert float(dx.abs().max()) == 0.0


@pytest.mark.parametrize("dims,m", [(D3, 4096), (D3, 131072), (NARROW, 65536)])
def test_atomic_flush_path_matches_oracle(dims, m):
    # mlpmk_bwd (every workgroup adds its partials with fp32 atomics) next to
    # the workspace path the other tests take.
    _, _, dws, dx, rdws, rdx = run_train(dims, m, seed=21, workspace=False)
    for i in range(len(dws)):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1} (atomics)")
    ok, err, _ = orc.allclose_report(dx.float().cpu().numpy(), rdx, 1e-2, 1e-2)
    assert ok, f"dx (atomics): {err}"


def test_workspace_and_atomic_paths_agree():
    # Same inputs through both reductions: equal up to fp32 summation order.
    x, ws = orc.make_inputs(D3, 65536, seed=5)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    dout = torch.ones((1, 128), dtype=torch.float16, device="cuda").expand(65536, 128)
    a = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    b = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    ops.bwd(xd, wd, hs, dout, a, workspace=True)
    ops.bwd(xd, wd, hs, dout, b, workspace=False)
    torch.cuda.synchronize()
    for i in range(3):
        scale = b[i].abs().max().item()
        assert torch.allclose(a[i], b[i], rtol=1e-5, atol=1e-6 * scale), f"dW{i + 1}"


def test_workspace_too_small_is_rejected():
    import ctypes
    from mlpmk import _lib
    x, ws = orc.make_inputs(D3, 4096, seed=6)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    dout = torch.ones((1, 128), dtype=torch.float16, device="cuda").expand(4096, 128)
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    need = ops.bwd_workspace_bytes(list(D3), 4096, False)
    assert need > 0 and need % (4 * 49152) == 0
    buf = torch.empty(need, dtype=torch.uint8, device="cuda")
    lib = _lib.get()
    pd, _k1 = _lib.int_array(list(D3))
    pw, _k2 = _lib.ptr_array([w.data_ptr() for w in wd])
    ps, _k3 = _lib.ptr_array([h.data_ptr() for h in hs])
    pg, _k4 = _lib.ptr_array([d.data_ptr() for d in dws])
    rc = lib.mlpmk_bwd_ws(3, pd, 1, xd.data_ptr(), pw, ps, dout.data_ptr(), 0, None, pg, buf.data_ptr(), need - 16,
                          4096, torch.cuda.current_stream().cuda_stream)
    assert rc == 1 and b"workspace_bytes" in lib.mlpmk_last_error()
    assert all(d.abs().max().item() == 0 for d in dws)  # nothing launched


@pytest.mark.parametrize("m", [4096, 131072])
def test_saturated_units_weight_gradients(m):
    # Columns of W1 drive their pre-activation to a constant z in -10 .. -20
    # (x[:, 0] = 1 and the column is z at row 0, 0 elsewhere), and three
    # columns of W2 drive theirs to ~-12 .. -25 (all weights -0.2 against
    # h1 ~ 0.7).  Their units saturate: h = softplus(z) ~ e^z, the derivative
    # sigma = 1 - e^-h ~ h is evaluated as -expm1(-h) in the kernel (the plain
    # 1 - exp(-h) has no correct digit below h ~ 1e-7), and dz = dh * sigma
    # is tiny.  Down to z ~ -12 every dW entry of those columns must meet
    # rtol 2e-2 against the oracle, with an atol scaled by the column's own
    # magnitude; below, dz is an fp16 subnormal (the wgrad MFMA operand, as
    # the reference's tl.dot operands are INPUT_DTYPE), and each entry must
    # stay within that rounding: |err| <= 2e-2 |ref| + 2^-24 * sum_r |a[r, i]|.
    dims = (128, 128, 128, 128)
    x, ws = orc.make_inputs(dims, m, seed=31)
    x[:, 0] = np.float16(1.0)
    zs = [-10.0, -11.0, -12.0, -14.0, -16.0, -18.0, -20.0]
    cols1 = list(range(3, 3 + len(zs)))
    for c, z in zip(cols1, zs):
        ws[0][:, c] = 0
        ws[0][0, c] = np.float16(z)
    cols2 = [40, 41, 42]
    for c in cols2:
        ws[1][:, c] = np.float16(-0.2)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    dout = torch.ones((1, 128), dtype=torch.float16, device="cuda").expand(m, 128)
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
    ops.bwd(xd, wd, hs, dout, dws, None)
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, _ = orc.backward(x, ws, ref_h, np.ones((m, 128), np.float32), need_dx=False)
    acts = [x.astype(np.float64), ref_h[0].astype(np.float64)]
    z2 = (ref_h[0].astype(np.float16).astype(np.float64) @ ws[1][:, cols2].astype(np.float64))
    assert z2.max() < -10.0, z2.max()
    for layer, cols, zcol in ((0, cols1, zs), (1, cols2, [None] * len(cols2))):
        got = dws[layer].cpu().numpy().astype(np.float64)
        ref = rdws[layer].astype(np.float64)
        asum = np.abs(acts[layer]).sum(axis=0)  # sum_r |a[r, i]| per input feature i
        for c, z in zip(cols, zcol):
            g, r = got[:, c], ref[:, c]
            assert np.abs(r).max() > 0, (layer, c)
            if z is not None and z >= -12.0:
                bound = 2e-2 * np.abs(r) + 2e-3 * np.abs(r).max()
                what = f"dW{layer + 1}[:, {c}] (z = {z}) per entry at rtol 2e-2"
            else:
                bound = 2e-2 * np.abs(r) + 2.0 ** -24 * asum
                what = f"dW{layer + 1}[:, {c}] (z = {z}) within the fp16-dz rounding bound"
            excess = np.abs(g - r) - bound
            assert excess.max() <= 0, f"{what}: worst excess {excess.max():.3g}, max|ref| {np.abs(r).max():.3g}"
    # and the matrix as a whole, as everywhere else
    for i in range(3):
        check_dw(dws[i].cpu().numpy(), rdws[i], f"saturated net dW{i + 1}")


# MLPMK_DOUT_SCALAR: the backward reads one element for every row and column.
# Every case is checked against the oracle (weight gradients with check_dw,
# dx at atol = rtol = 1e-2; bf16 at its own tolerances), and against the same
# value materialised as a broadcast row: bit for bit where the partials go
# through the workspace and the combine's fixed order (the atomic flush of
# small grids sums in any order).  The recomputing kernels (last stash entry
# None) and bf16 tensors take the same dout path: rows past M must not pick
# up the scalar (a recomputed h_{L-1} there is forced to zero).
def _check_dw_bf16(got, ref, what, n_layers):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    worst = np.max(np.abs(got - ref) - (4e-2 * np.abs(ref) + (n_layers + 1) * 1e-3 * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < 2e-2, f"{what}: worst excess {worst:.3g} (scale {scale:.3g}), rel frob {frob:.3g}"


@pytest.mark.parametrize("dims,m,with_dx,elem,recompute", [
    (D3, 131072 + 5, False, "f16", False),
    (D3, 4096, True, "f16", False),
    (D5, 65536, False, "f16", False),
    (NARROW, 100000, True, "f16", False),
    ((48, 96, 80, 10), 3000, True, "f16", False),
    (D3, 131072 + 5, False, "f16", True),
    (D3, 1000, True, "f16", True),
    (D5, 4097, False, "f16", True),
    (D3, 70001, True, "bf16", False),
    (D3, 4096, False, "bf16", True),
    (D5, 3000, True, "bf16", False),
])
def test_scalar_dout_matches_oracle_and_broadcast_row(dims, m, with_dx, elem, recompute):
    L = len(dims) - 1
    dt = torch.bfloat16 if elem == "bf16" else torch.float16
    x, ws = orc.make_inputs(dims, m, seed=23, elem=elem)
    xd = torch.from_numpy(x).cuda().to(dt)
    wd = [torch.from_numpy(w).cuda().to(dt) for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True, recompute=recompute)
    assert (hs[-1] is None) == recompute
    c = torch.full((), 0.75, dtype=dt, device="cuda")
    douts = [c.expand(m, dims[-1]), c.reshape(1, 1).expand(1, dims[-1]).contiguous().expand(m, dims[-1])]
    res = []
    for dout in douts:
        dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(L)]
        dx = torch.empty_like(xd) if with_dx else None
        ops.bwd(xd, wd, hs, dout, dws, dx)
        res.append((dws, dx))
    torch.cuda.synchronize()
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True, elem=elem)
    rdws, rdx = orc.backward(x, ws, ref_h, np.full((m, dims[-1]), 0.75, np.float32), need_dx=with_dx)
    (da, xa), (db, xb) = res
    for i in range(L):
        what = f"scalar dout dW{i + 1} {dims} M={m} {elem}{' recompute' if recompute else ''}"
        if elem == "bf16":
            _check_dw_bf16(da[i].cpu().numpy(), rdws[i], what, L)
        else:
            check_dw(da[i].cpu().numpy(), rdws[i], what)
    if with_dx:
        tol = 3e-2 if elem == "bf16" else 1e-2
        ok, err, excess = orc.allclose_report(xa.float().cpu().numpy(), rdx, tol, tol)
        assert ok, f"scalar dout dx {dims} M={m} {elem}: max err {err:.3g}, excess {excess:.3g}"
    deterministic = -(-m // 128) >= 128  # 128-row rounds: grids well above the 64-workgroup atomic cut
    for i, (a, b) in enumerate(zip(da, db)):
        if deterministic:
            assert torch.equal(a, b), f"dW{i + 1}"
        else:
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-6 * float(b.abs().max())), f"dW{i + 1}"
    if with_dx:
        assert torch.equal(xa, xb)
