"""HIP-graph capture of the drop-in paths on the GPU.

The library allocates nothing, records no memset and launches on the current
stream, so a whole training step of the weight-norm module (weight-norm
forward, forward megakernel with stash, ``out.sum()``, backward megakernel
with its partial-sum combine, weight-norm backward) and the inference
launcher can be captured into one graph each.  Every replay here gets fresh
inputs, eager work runs between replays, and each replay is checked against
an eager copy of the model on the same inputs.

With grids of 64 workgroups or more the backward reduces its partials in a
fixed order, so eager and replayed gradients are bitwise equal; below that
(M = 4096) the atomic flush leaves last-bit differences.
"""
import copy

import pytest
import torch

import fused_mlp
import kernel

pytestmark = pytest.mark.gpu


def _fresh_x(m, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(m, 128, device="cuda", generator=g).half()


def _eager_step(model, x):
    model.v_all.grad = None
    model.g_all.grad = None
    out = model(x)
    out.sum().backward()
    return out.detach().clone(), model.v_all.grad.clone(), model.g_all.grad.clone()


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
    exact = m >= 16384
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
        assert torch.equal(model.v_all.grad, ref[1]), f"step {r}: dv"
        assert torch.equal(model.g_all.grad, ref[2]), f"step {r}: dg"


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
