"""Hidden widths above 128 (up to 256): the streamed-weight forward
(``fwd_wide.hip``) and the two-pass backward (``bwd_tp.hip``: data gradients
with streamed fragments, weight gradients by 64 x 64 blocks) against the CPU
oracle, and training of the drop-in modules at H = 256 (output widths that
are not a multiple of 8 train through the library-GEMM fallback).

The reference's kernel compiles for any hidden width (constexpr tile loops,
/root/reference/kernel.py:60-123; its modules take H, README.md:62,68) and
lists larger H as the next step (mlp_fused.md:453-454).  Tolerances as for
the 128-wide kernels: outputs at atol = rtol = 1e-2 against the fp32 oracle
(kernel.py:110,117 round the hidden activations to fp16 as the kernels do);
weight gradients per entry within 2e-2 |ref| + 2e-3 max|ref| and relative
Frobenius 1e-2.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fused_mlp
import kernel
from mlpmk import ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-2

SHAPES = [
    ((128, 256, 256, 128), 4096),
    ((128, 256, 256, 128), 131072),
    ((128, 256, 256, 128), 257),       # ragged: one full round plus one row
    ((256, 256, 256, 256), 8192),
    ((128, 256, 128), 3000),           # 2 layers
    ((64, 256, 192, 100), 5001),       # runtime widths, output not a multiple of 8
    ((16, 144, 48, 3), 777),           # one hidden width above 128, tiny output
    ((128, 128, 129), 1024),           # only the output above 128
    ((256, 64, 200), 999),             # input above 128
    ((128, 256, 256, 256, 256, 128), 4096),  # 5 layers
    ((96, 208, 160, 256, 50), 2048),   # 4 layers
]


def _check(got, ref, what):
    ok, err, _ = orc.allclose_report(np.asarray(got, np.float64), ref, TOL, TOL)
    assert ok, f"{what}: max|err| {err}"


@pytest.mark.parametrize("dims,m", SHAPES)
def test_wide_forward_matches_oracle(dims, m):
    x, ws = orc.make_inputs(dims, m, seed=len(dims) * 100 + m % 97)
    out = ops.fwd(torch.from_numpy(x).cuda(), [torch.from_numpy(w).cuda() for w in ws])
    assert tuple(out.shape) == (m, dims[-1]) and out.dtype == torch.float16
    _check(out.float().cpu().numpy(), orc.forward(x, ws, round_hidden=True), f"{dims} M={m}")
    info = ops.fwd_launch_info(dims, m)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    # rounds of 8 waves (256 rows) from 256 x CUs rows, of 4 waves below
    nw = 8 if m >= 256 * cus else 4
    assert info == {"kernel": "persistent", "rows_per_block": 32, "waves": nw,
                    "grid": min(-(-m // (32 * nw)), cus), "wgs_per_cu": 1}
    assert kernel._mirror_policy(m, dims, cus) == (32, nw)


def test_wide_forward_at_one_million_rows_sampled():
    dims, m = (128, 256, 256, 128), 1 << 20
    x, ws = orc.make_inputs(dims, m, seed=7)
    out = ops.fwd(torch.from_numpy(x).cuda(), [torch.from_numpy(w).cuda() for w in ws])
    idx = np.random.default_rng(0).choice(m, 8192, replace=False)
    idx[:4] = [0, 255, 256, m - 1]  # round edges
    _check(out.float().cpu().numpy()[idx], orc.forward(x[idx], ws, round_hidden=True), "1M sampled")


def test_wide_forward_bf16():
    dims, m = (128, 256, 256, 128), 4096
    x, ws = orc.make_inputs(dims, m, seed=9, elem="bf16")
    xb = torch.from_numpy(x).cuda().bfloat16()
    wb = [torch.from_numpy(w).cuda().bfloat16() for w in ws]
    out = ops.fwd(xb, wb)
    assert out.dtype == torch.bfloat16
    ok, err, _ = orc.allclose_report(out.float().cpu().numpy(), orc.forward(x, ws, round_hidden=True, elem="bf16"),
                                     3e-2, 3e-2)
    assert ok, err


@pytest.mark.parametrize("dims,m", [((128, 256, 256, 128), 4096), ((64, 256, 192, 100), 777)])
def test_wide_stash_matches_oracle_hidden(dims, m):
    x, ws = orc.make_inputs(dims, m, seed=13)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out, hs = ops.fwd(xd, wd, stash=True)
    ref, hidden = orc.forward(x, ws, round_hidden=True, return_hidden=True)
    _check(out.float().cpu().numpy(), ref, "out")
    for i, (h, r) in enumerate(zip(hs, hidden)):
        _check(h.cpu().numpy(), r, f"h{i + 1}")
    assert torch.equal(ops.fwd(xd, wd), out)  # inference and training forward agree bit for bit


def test_wide_forward_large_preactivations_and_nonfinite_rows():
    # z past 88.7 (2^u overflows fp32): softplus(z) = z, as the reference's
    # threshold gives; a row holding inf or NaN makes only its own outputs
    # non-finite, although the kernel pads widths with zero weights.
    dims, m = (128, 256, 256, 128), 2048
    x, ws = orc.make_inputs(dims, m, seed=17)
    big = np.arange(m) % 61 == 0
    x[big] = (x[big].astype(np.float32) * 300.0).astype(np.float16)
    x[5, 3] = np.inf
    x[700, 0] = np.nan
    out = ops.fwd(torch.from_numpy(x).cuda(), [torch.from_numpy(w).cuda() for w in ws]).float().cpu().numpy()
    ref = orc.forward(x, ws, round_hidden=True)
    bad = np.zeros(m, bool)
    bad[[5, 700]] = True
    assert not np.isfinite(out[bad]).all(axis=1).any()
    assert np.isfinite(out[~bad]).all()
    assert np.abs(ref[big & ~bad]).max() > 100.0
    row_scale = np.abs(ref).max(axis=1, keepdims=True)
    err = np.abs(out[~bad] - ref[~bad])
    assert np.all(err <= TOL + TOL * np.abs(ref[~bad]) + TOL * row_scale[~bad] * big[~bad][:, None]), float(err.max())


# M = 4096: 4-wave rounds of 128 rows, one round per workgroup; M = 300,000:
# 8-wave rounds of 256 rows, 4-5 rounds per workgroup, large rows in first,
# middle and last rounds.
@pytest.mark.parametrize("m", [4096, 300000])
@pytest.mark.parametrize("stash", [False, True])
def test_wide_large_preactivations_up_to_the_fp16_limit(stash, m):
    # Identity weights padded to 256: out = softplus(softplus(x)) on the first
    # 128 features.  Past z = 88.7, 2^u overflows fp32 and softplus(z) = z
    # must come out, as the reference's z > 20 branch gives, up to the fp16
    # limit of its hidden h (kernel.py:108,110): h = 65,504 stays finite
    # (with hidden values carried at 1/2 of the base-2 value the rounding
    # of 65,504 * 1.44 / 2 gave an output of 65,520, which is inf in fp16).
    dims = (128, 256, 256, 128)
    z = np.array([88.0, 88.8, 89.0, 100.0, 200.0, 1000.0, 3.0e4, 4.6e4, 5.0e4, 65504.0], dtype=np.float32)
    rng = np.random.default_rng(23)
    x = (rng.standard_normal((m, 128)) * 0.5).astype(np.float16)
    rows = [3, 40, m - 1] + ([256 * 257 + 5, 256 * 600 + 255] if m > 200000 else [2000])
    for r in rows:
        x[r, : z.size] = z.astype(np.float16)
    ws = [np.eye(dims[i], dims[i + 1], dtype=np.float16) for i in range(3)]
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    res = ops.fwd(xd, wd, stash=stash)
    out = (res[0] if stash else res).float().cpu().numpy()
    idx = np.unique(np.concatenate([rows, rng.choice(m, min(m, 4096), replace=False)]))
    ref, ref_h = orc.forward(x[idx], ws, return_hidden=True)
    _check(out[idx], ref, "identity weights, large z")
    for r in rows:
        np.testing.assert_allclose(out[r, : z.size], z, rtol=2e-3)
    if stash:
        for i, h in enumerate(res[1]):
            ok, err, _ = orc.allclose_report(h.cpu().numpy()[idx], ref_h[i], 2e-3, 2e-3)
            assert ok, f"stash h{i + 1}: max|err| {err}"
        assert torch.equal(res[0], ops.fwd(xd, wd))


@pytest.mark.parametrize("m", [4096, 131072])
def test_wide_scaled_inputs_overflow_in_every_round(m):
    # x scaled so that a large share of pre-activations pass z = 88.7 in
    # every layer, in every round; every 7th row keeps its ordinary scale
    # and shares those rounds.
    dims = (128, 256, 256, 128)
    x, ws = orc.make_inputs(dims, m, seed=29)
    x = (x.astype(np.float32) * 300.0).astype(np.float16)
    small = np.zeros(m, dtype=bool)
    small[::7] = True
    x[small] = (x[small].astype(np.float32) / 300.0).astype(np.float16)
    out = ops.fwd(torch.from_numpy(x).cuda(), [torch.from_numpy(w).cuda() for w in ws]).float().cpu().numpy()
    ref = orc.forward(x, ws, round_hidden=True)
    assert np.isfinite(ref).all()
    _check(out[small], ref[small], "ordinary rows in exact rounds")
    big_err = np.abs(out[~small] - ref[~small]).max()
    assert big_err <= 2e-3 * np.abs(ref[~small]).max(), (big_err, np.abs(ref[~small]).max())


def test_launcher_wider_than_256_runs_layer_by_layer():
    dims, m = (128, 320, 320, 128), 1000
    x, ws = orc.make_inputs(dims, m, seed=23)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    assert not ops.fwd_supported(list(dims))
    out = kernel._fused_mlp_fwd(xd, *wd)
    assert out.dtype == torch.float16 and tuple(out.shape) == (m, 128)
    _check(out.float().cpu().numpy(), orc.forward(x, ws, round_hidden=True), "layer by layer, H = 320")


def test_wide_launcher_matches_model():
    dims, m = (128, 256, 256, 64), 4096
    x, ws = orc.make_inputs(dims, m, seed=19)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out = kernel._fused_mlp_fwd(xd, *wd)
    eager = kernel.Model()(xd.float(), *[w.float() for w in wd])
    _check(out.float().cpu().numpy(), eager.cpu().numpy(), "vs eager Model")
    assert kernel._pick_config(m, *dims)[::5] == (32, 4)  # 4-wave rounds below 256 x CUs rows


def _torch_ref(x16, ws16):
    x = x16.detach().cpu().double().requires_grad_(True)
    ws = [w.detach().cpu().double().requires_grad_(True) for w in ws16]
    a = x
    for i, w in enumerate(ws):
        a = a @ w
        if i < len(ws) - 1:
            a = F.softplus(a)
    a.sum().backward()
    return a.detach().numpy(), x.grad.numpy(), [w.grad.numpy() for w in ws]


def _check_grad(got, ref, what, k=1.0):
    # k scales every bound: 3 for bf16 (3 fewer significand bits than fp16;
    # the bf16 tests check outputs at 3e-2 where the fp16 ones use 1e-2)
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    worst = np.max(np.abs(got - ref) - k * (2e-2 * np.abs(ref) + 2e-3 * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < k * 1e-2, f"{what}: worst excess {worst:.3g}, rel frob {frob:.3g}"


@pytest.mark.parametrize("H,n_layers,out_f", [(256, 3, 128), (192, 5, 128), (256, 3, 100), (320, 3, 128), (512, 2, 64)])
def test_module_with_wide_hidden_trains(H, n_layers, out_f):
    # (out_features 100, not a multiple of 8: the library-GEMM fallback
    # backward; H = 320 and 512: no fused forward takes widths above 256,
    # so these run layer by layer -- fp32 library GEMMs, the library's fp32
    # softplus kernel, h rounded to fp16 between layers -- and train through
    # the fallback backward)
    from mlpmk import autograd as mag

    torch.manual_seed(3)
    model = fused_mlp.FusedMLPSoftplus(D=128, H=H, out_features=out_f, n_layers=n_layers).cuda().half()
    assert mag._fused_bwd_supported(tuple(model.dims)) == (out_f % 8 == 0 and H <= 256)
    assert mag._layerwise(tuple(model.dims), torch.float16) == (H > 256)
    x = torch.randn(4096, 128, device="cuda").half().requires_grad_(True)
    out = model(x)
    out.sum().backward()
    ref_out, ref_dx, ref_dws = _torch_ref(x, list(model.weights))
    _check(out.detach().float().cpu().numpy(), ref_out, "out")
    for i, w in enumerate(model.weights):
        _check_grad(w.grad.float().cpu().numpy(), ref_dws[i], f"dW{i + 1}")
    _check(x.grad.float().cpu().numpy(), ref_dx, "dx")


@pytest.mark.parametrize("wn", [False, True])
@pytest.mark.parametrize("D,H,out_f,n_layers", [(64, 96, 32, 7), (3, 64, 4, 7)])
def test_modules_no_fused_kernel_takes_train(wn, D, H, out_f, n_layers):
    # 7 layers (the fused kernels take 2..5; with a 3-wide input padding it
    # to 16 does not help): the forward runs layer by layer and the backward
    # is the fallback (weight norm: the library's single-launch kernels, up
    # to 8 layers).
    from mlpmk import autograd as mag

    torch.manual_seed(6)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls(D=D, H=H, out_features=out_f, n_layers=n_layers).cuda()
    assert mag._layerwise(tuple(model.dims), torch.float16)
    assert mag._input_pad(tuple(model.dims), torch.float16) == 0
    x = torch.randn(1500, D, device="cuda").half().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        out = model(x)
    assert out.dtype == torch.float16
    out.float().sum().backward()
    if wn:
        ws = [model.v(i).detach() * (model.g(i).detach() / model.v(i).detach().norm(dim=0)) for i in range(n_layers)]
        ws16 = [w.half() for w in ws]
    else:
        ws16 = [w.detach().half() for w in model.weights]
    ref_out, ref_dx, ref_dws = _torch_ref(x, ws16)
    _check(out.detach().float().cpu().numpy(), ref_out, "out")
    _check(x.grad.float().cpu().numpy(), ref_dx, "dx")
    if not wn:
        for i, w in enumerate(model.weights):
            _check_grad(w.grad.float().cpu().numpy(), ref_dws[i], f"dW{i + 1}")
    else:
        assert torch.isfinite(model.v_all.grad).all() and torch.isfinite(model.g_all.grad).all()


@pytest.mark.parametrize("wn", [False, True])
@pytest.mark.parametrize(
    "D,H,out_f,n_layers,dtype",
    [
        (3, 64, 4, 3, torch.float16),  # out 4: the library-GEMM fallback backward
        (3, 128, 16, 3, torch.float16),  # the fused backward
        (63, 128, 8, 2, torch.bfloat16),
        (5, 256, 16, 3, torch.float16),  # the streamed-weight forward, two-pass backward
        (3, 64, 16, 3, torch.float32),
    ],
)
def test_modules_padded_input_train(wn, D, H, out_f, n_layers, dtype):
    # An input width that is not a multiple of 16 (xyz of a neural field) is
    # zero-padded to the next one so that the fused kernels take the network;
    # dx and dW_1 come back at the caller's width.
    from mlpmk import autograd as mag

    torch.manual_seed(7)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls(D=D, H=H, out_features=out_f, n_layers=n_layers).cuda()
    if not wn:
        model = model.to(dtype)
    dims = tuple(model.dims)
    assert mag._layerwise(dims, dtype) and mag._input_pad(dims, dtype) == -D % 16
    x = torch.randn(1500, D, device="cuda").to(dtype).requires_grad_(True)
    out = model(x)
    assert out.dtype == dtype and tuple(out.shape) == (1500, out_f)
    with torch.no_grad():  # the inference launch, padded the same way
        torch.testing.assert_close(model(x), out.detach(), atol=1e-3, rtol=1e-3)
    out.float().sum().backward()
    assert x.grad.shape == x.shape
    if wn:
        ws = [(model.v(i) * (model.g(i) / model.v(i).norm(dim=0))).detach().to(dtype) for i in range(n_layers)]
    else:
        ws = [w.detach() for w in model.weights]
    ref_out, ref_dx, ref_dws = _torch_ref(x, ws)
    k = 3.0 if dtype == torch.bfloat16 else 1.0
    if dtype == torch.float32:
        ok, err, _ = orc.allclose_report(out.detach().double().cpu().numpy(), ref_out, 2e-3, 2e-3)
        assert ok, f"out: max|err| {err}"
    else:
        ok, err, _ = orc.allclose_report(out.detach().double().cpu().numpy(), ref_out, k * TOL, k * TOL)
        assert ok, f"out: max|err| {err}"
    _check_grad(x.grad.float().cpu().numpy(), ref_dx, "dx", k)
    if not wn:
        assert model.weights[0].grad.shape == (D, H)
        for i, w in enumerate(model.weights):
            _check_grad(w.grad.float().cpu().numpy(), ref_dws[i], f"dW{i + 1}", k)
    else:
        # dW_1 against the closed form through the weight-norm backward
        v0, g0 = model.v(0).detach().double().cpu(), model.g(0).detach().double().cpu()
        n0 = v0.norm(dim=0)
        dw0 = torch.from_numpy(ref_dws[0])
        dg0 = (dw0 * v0).sum(0) / n0
        dv0 = g0 / n0 * dw0 - (g0 * dg0 / n0**2) * v0
        _check_grad(model.v_all.grad[: D * H].view(D, H).double().cpu().numpy(), dv0.numpy(), "dv1", k)
        _check_grad(model.g_all.grad[:H].double().cpu().numpy(), dg0.numpy(), "dg1", k)


def test_padded_input_empty_batch():
    # M = 0 through the padded path: empty output, empty gradients.
    model = fused_mlp.FusedMLPSoftplus(D=3, H=64, out_features=16).cuda().half()
    x = torch.zeros(0, 3, device="cuda", dtype=torch.float16, requires_grad=True)
    out = model(x)
    assert out.shape == (0, 16)
    out.sum().backward()
    assert x.grad.shape == (0, 3)
    assert model.weights[0].grad.shape == (3, 64) and not model.weights[0].grad.any()


def test_launcher_padded_input():
    # kernel.py's launcher pads K1 the same way.
    torch.manual_seed(8)
    x = torch.randn(777, 3, device="cuda").half()
    ws = [(torch.randn(a, b, device="cuda") / a**0.5).half() for a, b in ((3, 128), (128, 128), (128, 64))]
    out = kernel._fused_mlp_fwd(x, *ws)
    assert out.shape == (777, 64) and out.dtype == torch.float16
    ref_out, _, _ = _torch_ref(x, ws)
    _check(out.float().cpu().numpy(), ref_out, "out")


def test_weight_norm_module_with_wide_hidden_trains():
    torch.manual_seed(4)
    model = fused_mlp.FusedMLPSoftplusWN(D=128, H=256, out_features=128).cuda()
    x = torch.randn(2048, 128, device="cuda").half()
    with torch.no_grad():
        out_inf = model(x)
    out = model(x)
    assert torch.equal(out.detach(), out_inf)
    out.sum().backward()
    assert torch.isfinite(model.v_all.grad).all() and torch.isfinite(model.g_all.grad).all()
    # against the oracle of one weight-norm training step
    dims = model.dims
    xs = x.cpu().numpy()
    w16, vs, gs = [], [], []
    for i in range(len(dims) - 1):
        v = model.v(i).detach().cpu().numpy()
        g = model.g(i).detach().cpu().numpy()
        w16.append(orc.wn_forward(v, g)[0].astype(np.float16))
        vs.append(v)
        gs.append(g)
    ref, hidden = orc.forward(xs, w16, return_hidden=True, round_hidden=True)
    _check(out.detach().float().cpu().numpy(), ref, "wn out")
    dws, _ = orc.backward(xs, w16, hidden, np.ones(dims[-1], np.float32), need_dx=False)
    dv, dg = zip(*[orc.wn_backward(dws[i], vs[i], gs[i]) for i in range(len(vs))])
    _check_grad(model.v_all.grad.cpu().numpy(), np.concatenate([d.reshape(-1) for d in dv]), "dv")
    _check_grad(model.g_all.grad.cpu().numpy(), np.concatenate(dg), "dg")


# The two-pass backward at widths above 128, through the C ABI (ops.bwd ->
# mlpmk_bwd_ws), against the oracle's closed-form backward on the oracle's
# own hidden activations (rounded to fp16 as the kernels' operands are).
def _check_dw(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    worst = np.max(np.abs(got - ref) - (2e-2 * np.abs(ref) + 2e-3 * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < 1e-2, f"{what}: worst excess {worst:.3g} (scale {scale:.3g}), rel frob {frob:.3g}"


@pytest.mark.parametrize("dims,m,with_dx,dout_mode", [
    ((128, 256, 256, 128), 4096, True, "scalar"),
    ((128, 256, 256, 128), 4096, False, "dense"),
    ((128, 256, 256, 128), 131072, False, "scalar"),
    ((128, 256, 256, 128), 131072, True, "dense"),
    ((256, 256, 256, 256), 8192, True, "dense"),
    ((128, 192, 256, 64), 4096, True, "row"),
    ((256, 64, 200), 999, True, "dense"),
    ((128, 256, 256, 256, 256, 128), 4096, True, "scalar"),
    ((96, 208, 160, 256, 48), 2048, True, "dense"),
])
def test_wide_two_pass_backward_matches_oracle(dims, m, with_dx, dout_mode):
    assert ops.bwd_supported(list(dims))
    x, ws = orc.make_inputs(dims, m, seed=m + len(dims))
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    rng = np.random.default_rng(m)
    if dout_mode == "scalar":
        dnp = np.full((m, dims[-1]), 0.5, np.float32)
        dout = torch.full((), 0.5, dtype=torch.float16, device="cuda").expand(m, dims[-1])
    elif dout_mode == "row":
        row = rng.standard_normal(dims[-1]).astype(np.float16)
        dnp = np.broadcast_to(row.astype(np.float32), (m, dims[-1]))
        dout = torch.from_numpy(row).cuda().reshape(1, -1).expand(m, dims[-1])
    else:
        d16 = rng.standard_normal((m, dims[-1])).astype(np.float16)
        dnp = d16.astype(np.float32)
        dout = torch.from_numpy(d16).cuda()
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    dx = torch.empty_like(xd) if with_dx else None
    ops.bwd(xd, wd, hs, dout, dws, dx)
    torch.cuda.synchronize()
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, rdx = orc.backward(x, ws, ref_h, dnp, need_dx=with_dx)
    for i in range(len(dws)):
        _check_dw(dws[i].cpu().numpy(), rdws[i], f"{dims} M={m} dW{i + 1}")
    if with_dx:
        _check(dx.float().cpu().numpy(), rdx, f"{dims} M={m} dx")


def test_wide_backward_needs_the_workspace():
    # The two-pass backward hands dz between its passes through the
    # workspace: mlpmk_bwd (none) refuses widths above 128.
    dims = (128, 256, 128)
    x, ws = orc.make_inputs(dims, 256, seed=1)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    _, hs = ops.fwd(xd, wd, stash=True)
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(2)]
    with pytest.raises(ops.MlpmkError, match="mlpmk_bwd_ws"):
        ops.bwd(xd, wd, hs, torch.ones((256, 128), dtype=torch.float16, device="cuda"), dws, workspace=False)
