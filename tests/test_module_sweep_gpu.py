"""A seeded sweep of the drop-in training modules on the GPU: the
``FusedMLPSoftplus`` / ``FusedMLPSoftplusWN`` constructors over random
``D, H, out_features, n_layers`` (/root/reference/README.md:62,68), inputs
of fp16, bf16 and fp32 (with and without autocast), one forward and one
backward each, against float64 autograd of the same network on the CPU.

The draws cover every route the modules take: the compiled and runtime-width
fused kernels, the streamed-weight forward and two-pass backward (H up to
256), input widths padded to a multiple of 16 (any D), and the
layer-by-layer path (H = 320, more than 5 layers, fp32 wider than 128).

The float64 reference rounds what the kernels round: W (and W = g v / ||v||
for weight norm) and every hidden activation to the network's element type
(straight through for the gradients, as the kernels' own backward treats
them).  Tolerances scale with that type: outputs at atol = rtol = 1e-2
(fp16), 3e-2 (bf16), 1e-3 (fp32); gradients per entry within
k (2e-2 |ref| + 2e-3 max(1, (L + 1) / 4) max|ref|) for an L-layer network
(the data gradient is rounded to the element type once per layer on its
way down, which the reference does not do) and relative Frobenius k 1e-2,
with k = 1, 3 and 0.1.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fused_mlp
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu

_TYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
_K = {"f16": 1.0, "bf16": 3.0, "f32": 0.1}


def _draw(n, seed=31):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        n_layers = int(rng.choice([2, 3, 3, 4, 5, 6, 7]))
        H = int(rng.choice([16, 48, 64, 96, 128, 128, 160, 256, 320]))
        D = int(rng.integers(1, 161)) if rng.random() < 0.5 else 16 * int(rng.integers(1, 9))
        out_f = int(rng.integers(1, 161)) if rng.random() < 0.5 else 8 * int(rng.integers(1, 17))
        x_type = str(rng.choice(["f16", "bf16", "f32"]))
        autocast = x_type == "f32" and rng.random() < 0.4  # fp32 module under fp16 autocast
        wn = bool(rng.random() < 0.5)
        m = int(rng.choice([1, 100, 3000, 20000]))
        cases.append((D, H, out_f, n_layers, x_type, autocast, wn, m))
    return cases


CASES = _draw(40)


def _id(c):
    D, H, out_f, n_layers, x_type, autocast, wn, m = c
    return f"D{D}_H{H}_o{out_f}_L{n_layers}_{x_type}{'_amp' if autocast else ''}{'_wn' if wn else ''}_M{m}"


def _check(got, ref, what, k):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    tol = 1e-2 * k
    ok, err, excess = orc.allclose_report(got, ref, tol, tol)
    assert ok, f"{what}: max|err| {err:.4g}, worst excess {excess:.4g}"


def _check_grad(got, ref, what, k, n_layers):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    floor = 2e-3 * max(1.0, (n_layers + 1) / 4)  # one rounding of the data gradient per layer
    worst = np.max(np.abs(got - ref) - k * (2e-2 * np.abs(ref) + floor * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < k * 1e-2, f"{what}: worst excess {worst:.3g}, rel frob {frob:.3g}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_random_module_step_matches_float64(case):
    D, H, out_f, n_layers, x_type, autocast, wn, m = case
    print(f"case {_id(case)}", flush=True)
    torch.manual_seed(sum(case[:4]) + m)
    cls = fused_mlp.FusedMLPSoftplusWN if wn else fused_mlp.FusedMLPSoftplus
    model = cls(D=D, H=H, out_features=out_f, n_layers=n_layers).cuda()
    xt = _TYPES[x_type]
    if not wn and not autocast:
        model = model.to(xt)  # parameters in the input's type (fp32 stays fp32)
    # the element type the network runs in: the autocast type, else x's
    et = "f16" if autocast else x_type
    dt = _TYPES[et]
    x = torch.randn(m, D, device="cuda").to(xt).requires_grad_(True)
    coef = torch.linspace(-1, 1, out_f, device="cuda")
    with torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
        out = model(x)
    assert out.shape == (m, out_f) and out.dtype == dt
    (out.float() * coef).sum().backward()

    # float64 reference on the CPU, rounding what the kernels round
    params = [p.detach().double().cpu().requires_grad_(True) for p in model.parameters()]
    dims = model.dims
    if wn:
        v_all, g_all = params
        ws, vo, go = [], 0, 0
        for i in range(n_layers):
            v = v_all[vo:vo + dims[i] * dims[i + 1]].reshape(dims[i], dims[i + 1])
            g = g_all[go:go + dims[i + 1]]
            ws.append((v * (g / v.norm(dim=0))).to(dt).double())
            vo += dims[i] * dims[i + 1]
            go += dims[i + 1]
    else:
        ws = [p.to(dt).double() for p in params]
    xr = x.detach().to(dt).double().cpu().requires_grad_(True)
    a = xr
    for i, w in enumerate(ws):
        a = a @ w
        if i < n_layers - 1:
            a = F.softplus(a).to(dt).double()
    (a * coef.double().cpu()).sum().backward()

    k = _K[et]
    _check(out.detach().double().cpu().numpy(), a.detach().numpy(), "out", k)
    assert x.grad is not None and x.grad.shape == x.shape and x.grad.dtype == xt
    _check_grad(x.grad.double().cpu().numpy(), xr.grad.numpy(), "dx", k, n_layers)
    for j, (p, r) in enumerate(zip(model.parameters(), params)):
        assert p.grad.shape == p.shape
        _check_grad(p.grad.double().cpu().numpy(), r.grad.numpy(), f"param {j} grad", k, n_layers)
