"""Forward megakernel parity on the GPU: HIP path (through the C ABI) vs the
CPU oracle on the same seeded inputs.

Tolerance: fp16 outputs within atol = rtol = 1e-2 of the fp32 CPU evaluation
(the reference's own gate, /root/reference/profile.py:92, and BASELINE.json's
north_star).  Large M is checked on a random sample of rows (rows are
independent) plus exact row-permutation equivariance.
"""
import numpy as np
import pytest
import torch

from oracle import mlp_oracle as orc
import mlpmk
from mlpmk import ops

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-2


def _to_dev(x, ws):
    return torch.from_numpy(x).cuda(), [torch.from_numpy(w).cuda() for w in ws]


def _check(out, ref, what):
    ok, err, excess = orc.allclose_report(out, ref, ATOL, RTOL)
    assert ok, f"{what}: max|err|={err:.4g}, worst excess over atol+rtol*|ref| = {excess:.4g}"
    return err


def test_library_is_the_native_one():
    assert ops.library_path().endswith("libmlpmk.so")
    lib = mlpmk._lib.get()
    assert lib.mlpmk_version() >= 100


@pytest.mark.parametrize("m", [256, 64, 128, 512, 1024, 2048, 4096])
def test_3l128_latency_sweep_sizes(m):
    x, ws = orc.make_inputs((128, 128, 128, 128), m, seed=0)
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    _check(out, orc.forward(x, ws), f"3L-128 M={m}")


@pytest.mark.parametrize("m", [1, 31, 63, 65, 255, 257, 1000, 4097])
def test_3l128_ragged_tails(m):
    x, ws = orc.make_inputs((128, 128, 128, 128), m, seed=m)
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    _check(out, orc.forward(x, ws), f"3L-128 M={m}")


def test_3l128_matches_fp16_rounding_variant_tightly():
    # Against the oracle that rounds hidden activations to fp16 like the
    # reference megakernel (kernel.py:110,117) the error is a few fp16 ulps.
    x, ws = orc.make_inputs((128, 128, 128, 128), 4096, seed=3)
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    ref = orc.forward(x, ws, round_hidden=True)
    ok, err, _ = orc.allclose_report(out, ref, 4e-3, 4e-3)
    assert ok, err


def test_m0_is_noop():
    x = torch.empty((0, 128), dtype=torch.float16, device="cuda")
    ws = [torch.randn(128, 128, device="cuda").half() for _ in range(3)]
    out = ops.fwd(x, ws)
    assert out.shape == (0, 128)


def test_5l128_forward():
    x, ws = orc.make_inputs((128,) * 6, 65536, seed=0)
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    _check(out, orc.forward(x, ws), "5L-128 M=65536")


@pytest.mark.parametrize("m", [64, 1000, 65536])
def test_narrow_forward(m):
    x, ws = orc.make_inputs((32, 64, 64, 16), m, seed=0, x_dist="uniform")
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    _check(out, orc.forward(x, ws), f"narrow M={m}")


@pytest.mark.parametrize(
    "dims,m,uniform",
    [
        ((128, 128, 128, 128), 40000, False),  # 8-wave workgroups (1024 < blocks <= 2048)
        ((128,) * 6, 20000, False),  # 4-wave workgroups (625 blocks)
        ((32, 64, 64, 16), 100000, True),  # 8-wave workgroups, 64-row blocks
    ],
)
def test_small_batch_launch_shapes(dims, m, uniform):
    x, ws = orc.make_inputs(dims, m, seed=1, x_dist="uniform" if uniform else "normal")
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    _check(out, orc.forward(x, ws), f"{dims} M={m}")


@pytest.mark.parametrize(
    "dims,sizes,uniform",
    [
        ((128, 128, 128, 128), (4096, 16384, 65536, 1048576), False),
        ((128,) * 6, (4096, 20000, 65536, 1048576), False),
        ((32, 64, 64, 16), (4096, 40000, 131072, 4194304), True),
    ],
)
def test_launch_shape_does_not_change_results(dims, sizes, uniform):
    # The host picks the feature-split kernel (a block or two per CU), or 4-,
    # 8- or NW-wave workgroups of the one-block-per-wave kernel, by batch size
    # (the sizes here take each in turn); a row's result must not depend on
    # which kernel computed it.
    x, ws = _device_inputs(dims, max(sizes), seed=2, uniform=uniform)
    outs = [ops.fwd(x[:m].contiguous(), ws) for m in sizes]
    n = min(sizes)
    for m, o in zip(sizes[1:], outs[1:]):
        assert torch.equal(o[:n], outs[0]), f"{dims}: rows of M={m} differ from M={sizes[0]}"


def _device_inputs(dims, m, seed, uniform=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    if uniform:
        x = (torch.rand((m, dims[0]), generator=g, device="cuda") * 2 - 1).half()
    else:
        x = torch.randn((m, dims[0]), generator=g, device="cuda").half()
    ws = [
        (torch.randn((dims[i], dims[i + 1]), generator=g, device="cuda") / dims[i] ** 0.5).half()
        for i in range(len(dims) - 1)
    ]
    return x, ws


@pytest.mark.parametrize(
    "dims,m,uniform",
    [
        ((128, 128, 128, 128), 1048576, False),
        ((128,) * 6, 1048576, False),
        ((32, 64, 64, 16), 4194304, True),
    ],
)
def test_full_size_sampled_rows_and_permutation(dims, m, uniform):
    x, ws = _device_inputs(dims, m, seed=0, uniform=uniform)
    out = ops.fwd(x, ws)
    # 1) 4096 random rows against the oracle
    idx = torch.randperm(m, device="cuda")[:4096]
    xs = x[idx].cpu().numpy()
    wn = [w.cpu().numpy() for w in ws]
    _check(out[idx].float().cpu().numpy(), orc.forward(xs, wn), f"{dims} M={m} sampled")
    # 2) row independence: a permuted input gives the permuted output, bit for bit
    perm = torch.randperm(m, device="cuda")
    out_p = ops.fwd(x[perm].contiguous(), ws)
    assert torch.equal(out_p, out[perm])
    # 3) the last rows (tail of the persistent walk) are right too
    xs = x[-300:].cpu().numpy()
    _check(out[-300:].float().cpu().numpy(), orc.forward(xs, wn), f"{dims} M={m} last rows")


def test_stash_matches_hidden_activations():
    x, ws = orc.make_inputs((128, 128, 128, 128), 3000, seed=5)
    xd, wd = _to_dev(x, ws)
    out, hs = ops.fwd(xd, wd, stash=True)
    ref, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    _check(out.float().cpu().numpy(), ref, "stash-mode out")
    for i, (h, rh) in enumerate(zip(hs, ref_h)):
        ok, err, _ = orc.allclose_report(h.cpu().numpy(), rh, 2e-3, 2e-3)
        assert ok, f"h{i + 1}: {err}"
    out2 = ops.fwd(xd, wd)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("m,recompute", [(131072 + 77, False), (131072 + 77, True), (40000 + 5, False)])
def test_stash_rows_of_the_persistent_kernels(m, recompute):
    # M = 131149 runs the 8-wave persistent training forward, whose stash
    # rows leave through the LDS staging tile (ragged last block); M = 40005
    # the 8-wave kernel at ~5 blocks per CU.  With recompute the last stash
    # entry is not requested.
    info = ops.fwd_launch_info((128, 128, 128, 128), m, stash=True)
    assert (info["kernel"], info["waves"]) == ("persistent", 8), info
    x, ws = orc.make_inputs((128, 128, 128, 128), m, seed=7)
    xd, wd = _to_dev(x, ws)
    out, hs = ops.fwd(xd, wd, stash=True, recompute=recompute)
    ref, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    _check(out.float().cpu().numpy(), ref, f"stash-mode out M={m}")
    assert torch.equal(out, ops.fwd(xd, wd))
    for i, h in enumerate(hs):
        if h is None:
            assert recompute and i == len(hs) - 1
            continue
        got = h.cpu().numpy()
        ok, err, _ = orc.allclose_report(got, ref_h[i], 2e-3, 2e-3)
        assert ok, f"h{i + 1} M={m}: {err}"
    # Every element of a requested entry is written (over a canary fill).
    canary = torch.full((m, 128), 7.0, device="cuda")
    ops.fwd_into(xd, wd, torch.empty_like(out), [canary, None])
    assert torch.equal(canary, hs[0])


def test_threshold_edges_through_identity_weights():
    # W1 = W2 = I makes out = softplus(softplus(x)) @ W3; with W3 = I the
    # output is the activation itself on chosen pre-activations, including the
    # threshold neighbourhood of kernel.py:108.
    z = np.array([-100, -20, -5, -1, 0, 0.5, 1, 5, 19.99, 20, 20.01, 30, 60], dtype=np.float32)
    x = np.zeros((64, 128), dtype=np.float16)
    x[:, : z.size] = z.astype(np.float16)
    eye = np.eye(128, dtype=np.float16)
    xd, wd = _to_dev(x, [eye, eye, eye])
    out = ops.fwd(xd, wd).float().cpu().numpy()
    ref = orc.forward(x, [eye, eye, eye])
    _check(out, ref, "identity-weight softplus(softplus(z))")
    assert abs(out[0, 4] - np.log(3.0)) < 2e-3  # z = 0: softplus(softplus(0)) = log(1 + 2)


# M = 256 runs the feature-split kernel, M = 16384 the one-block-per-wave
# one, M = 131072 the persistent 12-wave one (3 waves per SIMD).
@pytest.mark.parametrize("m", [256, 16384, 131072])
@pytest.mark.parametrize("stash", [False, True])
def test_large_preactivations_take_the_exact_path(stash, m):
    # Past z = 88.7 the kernel's direct softplus form overflows (2^u in base-2
    # units); such blocks are recomputed exactly and must give softplus(z) = z,
    # the reference's z > 20 branch (kernel.py:108), up to the fp16 limit of
    # the reference's hidden h (kernel.py:110).  Large rows sit among ordinary
    # ones inside the same 32-row blocks, and only some blocks have any.
    z = np.array([88.0, 88.8, 89.0, 100.0, 200.0, 1000.0, 3.0e4, 4.6e4, 5.0e4, 65504.0], dtype=np.float32)
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((m, 128)) * 0.5).astype(np.float16)
    rows = (3, 40, 41, 200)  # blocks 0, 1 and 6 of eight
    for r in rows:
        x[r, : z.size] = z.astype(np.float16)
    eye = np.eye(128, dtype=np.float16)
    xd, wd = _to_dev(x, [eye, eye, eye])
    res = ops.fwd(xd, wd, stash=stash)
    out = (res[0] if stash else res).float().cpu().numpy()
    ref, ref_h = orc.forward(x, [eye, eye, eye], return_hidden=True)
    _check(out, ref, "identity weights, large z")
    for r in rows:
        np.testing.assert_allclose(out[r, : z.size], z, rtol=2e-3)
    if stash:
        for i, h in enumerate(res[1]):
            ok, err, _ = orc.allclose_report(h.cpu().numpy(), ref_h[i], 2e-3, 2e-3)
            assert ok, f"stash h{i + 1}: max|err| {err}"


@pytest.mark.parametrize("m", [4096, 20000, 131072])
@pytest.mark.parametrize("dims,stash", [((128, 128, 128, 128), False), ((128, 128, 128, 128), True),
                                        ((128,) * 6, False), ((32, 64, 64, 16), False)])
def test_scaled_inputs_overflow_many_blocks(dims, stash, m):
    # x scaled so that ~30 % of pre-activations exceed z = 88.7 in every
    # layer and every block takes the exact path; every 7th row keeps its
    # ordinary scale and shares those blocks.
    x, ws = orc.make_inputs(dims, m, seed=21)
    x = (x.astype(np.float32) * 300.0).astype(np.float16)
    small = np.zeros(len(x), dtype=bool)
    small[::7] = True
    x[small] = (x[small].astype(np.float32) / 300.0).astype(np.float16)
    xd, wd = _to_dev(x, ws)
    res = ops.fwd(xd, wd, stash=stash)
    out = (res[0] if stash else res).float().cpu().numpy()
    # Hidden activations reach ~1.5e3, where one fp16 ulp is 1.0: compare
    # with the oracle that rounds them to fp16 like the reference kernel
    # (kernel.py:110,117), with a bound scaled to the output range for the
    # large rows and the usual one for the ordinary rows.
    ref = orc.forward(x, ws, round_hidden=True)
    assert np.isfinite(ref).all()
    _check(out[small], ref[small], f"{dims} ordinary rows in exact-path blocks")
    big_err = np.abs(out[~small] - ref[~small]).max()
    assert big_err <= 2e-3 * np.abs(ref[~small]).max(), (big_err, np.abs(ref[~small]).max())
    if stash:
        assert torch.equal(res[0], ops.fwd(xd, wd))


@pytest.mark.parametrize("m", [128, 16384, 131072])
def test_inf_and_nan_inputs_propagate_like_the_oracle(m):
    # inf * 0 inside the products gives NaN, as in the reference's fp32 dot;
    # rows without non-finite inputs are unaffected.
    x, ws = orc.make_inputs((128, 128, 128, 128), m, seed=4)
    x[5, 7] = np.inf
    x[70, 0] = -np.inf
    x[99, 3] = np.nan
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        ref = orc.forward(x, ws)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    fin = np.isfinite(ref).all(axis=1)
    assert fin.sum() == m - 3
    _check(out[fin], ref[fin], "finite rows next to non-finite ones")


@pytest.mark.parametrize("m", [256, 16384, 131072])
@pytest.mark.parametrize("stash", [False, True])
def test_overflow_into_negative_weight_row_is_not_absorbed(stash, m):
    # The fast softplus form overflows to +inf for z >= 88.7.  Here hidden
    # unit k of h1 overflows in a few rows and row k of W2 is strictly
    # negative, so in the fast form every pre-activation of layer 2 of those
    # rows is -inf, and softplus(-inf) = 0 would hide the overflow from any
    # test of the layer-2 activations.  The exact value is far from 0:
    # h1[k] = z = 100, z2 = 100 * (-1e-3) + (other terms) = O(1).  The kernel
    # must detect the overflow (the -inf pre-activations are non-finite) and
    # recompute those blocks exactly.
    rng = np.random.default_rng(5)
    k = 17
    x = (rng.standard_normal((m, 128)) * 0.5).astype(np.float16)
    rows = [1, 33, m - 2]
    for r in rows:
        x[r, k] = np.float16(100.0)
    w1 = np.eye(128, dtype=np.float16)
    w2 = (rng.standard_normal((128, 128)) / np.sqrt(128)).astype(np.float16)
    w2[k, :] = np.float16(-1e-3)
    w3 = (rng.standard_normal((128, 128)) / np.sqrt(128)).astype(np.float16)
    ws = [w1, w2, w3]
    xd, wd = _to_dev(x, ws)
    res = ops.fwd(xd, wd, stash=stash)
    out = (res[0] if stash else res).float().cpu().numpy()
    sel = np.array(sorted(set(rows) | set(range(0, m, max(1, m // 2048)))))
    ref = orc.forward(x[sel], ws)
    _check(out[sel], ref, "overflow feeding a negative weight row")
    # An absorbed overflow would leave h2 = 0 and out = 0 in those rows; the
    # exact outputs are O(1), so the check above tells the two apart.
    assert np.abs(orc.forward(x[rows], ws)).max(axis=1).min() > 0.5


def test_zero_first_layer_closed_form():
    x, ws = orc.make_inputs((128, 128, 128, 128), 512, seed=1)
    ws[0] = np.zeros_like(ws[0])
    xd, wd = _to_dev(x, ws)
    out = ops.fwd(xd, wd).float().cpu().numpy()
    w2 = ws[1].astype(np.float64)
    w3 = ws[2].astype(np.float64)
    h2 = np.log1p(np.exp(np.log(2.0) * w2.sum(axis=0)))
    row = h2 @ w3
    _check(out, np.broadcast_to(row, out.shape), "W1 = 0 closed form")
