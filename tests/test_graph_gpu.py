"""HIP-graph capture of the drop-in paths on the GPU.

The library allocates nothing, records no memset and launches on the current
stream, so a whole training step of the weight-norm module (weight-norm
forward, forward megakernel with stash, ``out.sum()``, backward megakernel
with its partial-sum combine, weight-norm backward) and the inference
launcher can be captured into one graph each.  Every replay here gets fresh
inputs, eager work runs between replays, and each replay is checked against
an eager copy of the model on the same inputs and against the CPU oracle
(outputs at atol = rtol = 1e-2; weight-norm gradients per entry within
2e-2 |ref| + 2e-3 max|ref| and relative Frobenius 1e-2).

Above 16,384 rows the 16-bit backward is the one-pass megakernel, whose
partial sums meet in a fixed order, so eager and replayed gradients are
bitwise equal; up to 16,384 rows the two-pass backward adds its weight-
gradient tiles with fp32 atomics, which leaves last-bit differences.
"""
import copy

import numpy as np
import pytest
import torch

import fused_mlp
import kernel
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu

# Batches up to this many rows take the two-pass backward (fp32 atomics in its
# weight-gradient pass; MLPMK_TP_MAX_ROWS in bwd.hip).
TWO_PASS_MAX_ROWS = 16384


def _fresh_x(m, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(m, 128, device="cuda", generator=g).half()


def _eager_step(model, x):
    model.v_all.grad = None
    model.g_all.grad = None
    out = model(x)
    out.sum().backward()
    return out.detach().clone(), model.v_all.grad.clone(), model.g_all.grad.clone()


def _oracle_wn_step(x, model):
    """CPU oracle of one weight-norm training step (loss = out.sum()): the
    forward on the fp16-rounded W = g v / ||v|| the kernels use, the
    closed-form backward from the fp32 activations, the weight-norm chain
    rule; returns out, dv_all, dg_all."""
    dims = model.dims
    xs = x.cpu().numpy()
    w16, vs, gs = [], [], []
    for i in range(len(dims) - 1):
        v = model.v(i).detach().cpu().numpy()
        g = model.g(i).detach().cpu().numpy()
        w16.append(orc.wn_forward(v, g)[0].astype(np.float16))
        vs.append(v)
        gs.append(g)
    out, hidden = orc.forward(xs, w16, return_hidden=True)
    dws, _ = orc.backward(xs, w16, hidden, np.ones(dims[-1], np.float32), need_dx=False)
    dv, dg = zip(*[orc.wn_backward(dws[i], vs[i], gs[i]) for i in range(len(vs))])
    return out, np.concatenate([d.reshape(-1) for d in dv]), np.concatenate(dg)


def _check_oracle(got, ref, what, grad):
    got = got.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, np.float64)
    if not grad:
        ok, err, _ = orc.allclose_report(got, ref, 1e-2, 1e-2)
        assert ok, f"{what}: max|err| {err}"
        return
    scale = np.abs(ref).max()
    worst = np.max(np.abs(got - ref) - (2e-2 * np.abs(ref) + 2e-3 * scale))
    frob = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert worst <= 0 and frob < 1e-2, f"{what}: worst excess {worst:.3g}, rel frob {frob:.3g}"


def _same(got, ref, exact, what):
    if exact:
        assert torch.equal(got, ref), what
    else:
        torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-6 * ref.abs().max().item(), msg=what)


@pytest.mark.parametrize("m", [4096, 16384, 131072])
def test_whole_training_step_graph(m):
    # out.sum() records a memset (torch's reduction) besides its kernel; the
    # replays below, each checked against eager with eager work in between,
    # are what keeps it inside the graph.
    torch.manual_seed(0)
    model = fused_mlp.FusedMLPSoftplusWN().cuda()
    ref_model = copy.deepcopy(model)
    static_x = _fresh_x(m, 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            _eager_step(model, static_x)
    torch.cuda.current_stream().wait_stream(side)
    model.v_all.grad = None
    model.g_all.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = model(static_x)
        static_out.sum().backward()
    static_dv, static_dg = model.v_all.grad, model.g_all.grad
    exact = m > TWO_PASS_MAX_ROWS
    for r in range(4):
        static_x.copy_(_fresh_x(m, 100 + r))
        graph.replay()
        torch.cuda.synchronize()
        got = (static_out.clone(), static_dv.clone(), static_dg.clone())
        ref = _eager_step(ref_model, static_x.clone())  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(got[0], ref[0]), f"replay {r}: out"
        _same(got[1], ref[1], exact, f"replay {r}: dv")
        _same(got[2], ref[2], exact, f"replay {r}: dg")
        o_out, o_dv, o_dg = _oracle_wn_step(static_x, ref_model)
        _check_oracle(got[0], o_out, f"replay {r}: out vs oracle", grad=False)
        _check_oracle(got[1], o_dv, f"replay {r}: dv vs oracle", grad=True)
        _check_oracle(got[2], o_dg, f"replay {r}: dg vs oracle", grad=True)


def _fresh_x_d(m, seed, d):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(m, d, device="cuda", generator=g).half()


@pytest.mark.parametrize("m", [4096, 131072])
@pytest.mark.parametrize("kind", ["fp32", "h256", "d3"])
def test_training_step_graph_two_pass_shapes(kind, m):
    # The weight-norm module with fp32 tensors (bf16 hi/lo split operands)
    # and with hidden width 256: both train through the two-pass backward at
    # every M (dz through the workspace, weight gradients written by atomics
    # after the data-gradient pass cleared dW).  "d3": a 3-wide input, padded
    # inside the step to 16 columns (torch's pad kernels captured with the
    # library's).  Replays with fresh inputs and eager work in between, each
    # against an eager copy of the model.
    torch.manual_seed(1)
    if kind == "fp32":
        model = fused_mlp.FusedMLPSoftplusWN()
    elif kind == "h256":
        model = fused_mlp.FusedMLPSoftplusWN(H=256)
    else:
        model = fused_mlp.FusedMLPSoftplusWN(D=3, out_features=16)
    model = model.cuda()
    ref_model = copy.deepcopy(model)
    dt = torch.float32 if kind == "fp32" else torch.float16
    width = 3 if kind == "d3" else 128
    static_x = _fresh_x_d(m, 0, width).to(dt)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            _eager_step(model, static_x)
    torch.cuda.current_stream().wait_stream(side)
    model.v_all.grad = None
    model.g_all.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = model(static_x)
        static_out.sum().backward()
    static_dv, static_dg = model.v_all.grad, model.g_all.grad
    assert static_out.dtype == dt and static_dv.dtype == torch.float32
    for r in range(3):
        static_x.copy_(_fresh_x_d(m, 200 + r, width).to(dt))
        graph.replay()
        torch.cuda.synchronize()
        got = (static_out.clone(), static_dv.clone(), static_dg.clone())
        ref = _eager_step(ref_model, static_x.clone())  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(got[0], ref[0]), f"{kind} replay {r}: out"
        _same(got[1], ref[1], False, f"{kind} replay {r}: dv")
        _same(got[2], ref[2], False, f"{kind} replay {r}: dg")


def test_make_graphed_callables_training():
    m = 16384
    torch.manual_seed(1)
    model = fused_mlp.FusedMLPSoftplusWN().cuda()
    ref_model = copy.deepcopy(model)
    graphed = torch.cuda.make_graphed_callables(model, (_fresh_x(m, 0),))
    for r in range(3):
        x = _fresh_x(m, 200 + r)
        model.v_all.grad = None
        model.g_all.grad = None
        out = graphed(x)
        out.sum().backward()
        ref = _eager_step(ref_model, x)
        torch.cuda.synchronize()
        assert torch.equal(out.detach(), ref[0]), f"step {r}: out"
        _same(model.v_all.grad, ref[1], m > TWO_PASS_MAX_ROWS, f"step {r}: dv")
        _same(model.g_all.grad, ref[2], m > TWO_PASS_MAX_ROWS, f"step {r}: dg")
        o_out, o_dv, o_dg = _oracle_wn_step(x, ref_model)
        _check_oracle(out, o_out, f"step {r}: out vs oracle", grad=False)
        _check_oracle(model.v_all.grad, o_dv, f"step {r}: dv vs oracle", grad=True)
        _check_oracle(model.g_all.grad, o_dg, f"step {r}: dg vs oracle", grad=True)


@pytest.mark.parametrize("m", [64, 4096, 65536])
def test_inference_launcher_graph(m):
    torch.manual_seed(2)
    ws = [(torch.randn(128, 128, device="cuda") / 128 ** 0.5).half() for _ in range(3)]
    static_x = _fresh_x(m, 0)
    kernel._fused_mlp_fwd(static_x, *ws)  # first call outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = kernel._fused_mlp_fwd(static_x, *ws)
    for r in range(4):
        static_x.copy_(_fresh_x(m, 300 + r))
        graph.replay()
        ref = kernel._fused_mlp_fwd(static_x.clone(), *ws)
        torch.cuda.synchronize()
        assert torch.equal(static_out, ref), f"replay {r}"
        o_out = orc.forward(static_x.cpu().numpy(), [w.cpu().numpy() for w in ws])
        _check_oracle(static_out, o_out, f"replay {r} vs oracle", grad=False)
