"""Batches past 2^32 tensor elements: 40,000,037 rows of the 3-layer 128-wide
network (x alone is 5.1 G fp16 elements, the fp32 stash 10.2 G), as the
288 GB of an MI355X hold them.

Row offsets inside the kernels are 64-bit; these tests run the forward, the
training forward and the one-pass backward (fp16), the streamed-weight
forward and training forward with the two-pass backward (hidden width 256),
and the fp32 training forward and two-pass backward over such a batch on
the GPU, and check rows on both sides of element 2^32 (row 2^25) against
the CPU oracle.
The weight gradient sums all 40 M rows, which the oracle cannot redo in a
test's time, so it is checked through a size-independent identity instead:
dW over the whole batch equals dW over its first half plus dW over its
second half (each half launched separately, with its own base pointers and
small row indices), to fp32 summation-order rounding.  Tolerances as for the
other forward tests: atol = rtol = 1e-2 against the fp32 oracle for 16-bit
tensors (kernel.py:110,117 round the hidden activations to fp16 as the
kernels do); 2e-4 of each row's scale against the fp64 oracle for fp32
tensors.
"""
import numpy as np
import pytest
import torch

from mlpmk import ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu

M = 40_000_037
DIMS = (128, 128, 128, 128)
EDGE = 1 << 25  # first row whose x elements start past 2^32


def _rows(m):
    rng = np.random.default_rng(3)
    fixed = [0, 1, EDGE - 1, EDGE, EDGE + 1, m // 2 - 1, m // 2, m - 2, m - 1]
    return np.unique(np.concatenate([fixed, rng.choice(m, 4096, replace=False)]))


def _check(got, ref, what, tol=1e-2):
    ok, err, _ = orc.allclose_report(np.asarray(got, np.float64), ref, tol, tol)
    assert ok, f"{what}: max|err| {err}"


def _check_dw(dw, dwa, dwb, h_last, dout_row):
    """dW over the whole batch against dW over its halves, and the last
    layer's against its closed form: with one dout row broadcast over the
    batch, dW_{L-1} = (sum over rows of h_{L-1}) (outer) dout_row, the column
    sums taken in float64 on the GPU."""
    for i in range(len(dw)):
        full = dw[i].double().cpu()
        parts = (dwa[i].double() + dwb[i].double()).cpu()
        assert torch.isfinite(full).all()
        rel = ((full - parts).norm() / full.norm()).item()
        print(f"dW{i + 1}: |full - (a + b)| / |full| = {rel:.3g}")
        assert rel < 1e-4, (i, rel)
    exact = torch.outer(h_last.double().sum(0), dout_row.double()).cpu()
    for name, got in (("full", dw[-1].double().cpu()), ("halves", (dwa[-1].double() + dwb[-1].double()).cpu())):
        rel = ((got - exact).norm() / exact.norm()).item()
        print(f"dW{len(dw)} {name}: |got - exact| / |exact| = {rel:.3g}")
        assert rel < 3e-5, (name, rel)


@pytest.fixture(scope="module")
def batch():
    _, ws = orc.make_inputs(DIMS, 1, seed=31)
    g = torch.Generator(device="cuda").manual_seed(31)
    x = torch.randn((M, DIMS[0]), generator=g, device="cuda", dtype=torch.float16)
    wd = [torch.from_numpy(w).cuda() for w in ws]
    idx = _rows(M)
    xs = x[torch.from_numpy(idx).cuda()].cpu().numpy()
    yield x, wd, ws, idx, xs
    del x
    torch.cuda.empty_cache()


def test_forward_past_2_32_elements(batch):
    x, wd, ws, idx, xs = batch
    out = ops.fwd(x, wd)
    got = out[torch.from_numpy(idx).cuda()].float().cpu().numpy()
    del out
    _check(got, orc.forward(xs, ws, round_hidden=True), "sampled rows")


def test_training_forward_and_backward_past_2_32_elements(batch):
    x, wd, ws, idx, xs = batch
    out, hs = ops.fwd(x, wd, stash=True)
    ti = torch.from_numpy(idx).cuda()
    ref, ref_h = orc.forward(xs, ws, round_hidden=True, return_hidden=True)
    _check(out[ti].float().cpu().numpy(), ref, "sampled rows")
    for i, h in enumerate(hs):
        _check(h[ti].cpu().numpy(), ref_h[i], f"stash h{i + 1}")
    del out

    g = torch.Generator(device="cuda").manual_seed(32)
    dout = torch.randn((1, DIMS[-1]), generator=g, device="cuda", dtype=torch.float16).expand(M, DIMS[-1])
    dw = [torch.empty((DIMS[i], DIMS[i + 1]), device="cuda") for i in range(3)]
    ops.bwd(x, wd, hs, dout, dw, accumulate=False)
    half = M // 2
    dwa = [torch.empty_like(d) for d in dw]
    dwb = [torch.empty_like(d) for d in dw]
    ops.bwd(x[:half], wd, [h[:half] for h in hs], dout[:half], dwa, accumulate=False)
    ops.bwd(x[half:], wd, [h[half:] for h in hs], dout[half:], dwb, accumulate=False)
    _check_dw(dw, dwa, dwb, hs[-1], dout[0])


def test_wide_forward_past_2_32_elements(batch):
    # Hidden width 256: the streamed-weight forward, rounds of 256 rows.
    x, _, _, idx, xs = batch
    dims = (128, 256, 256, 128)
    _, ws = orc.make_inputs(dims, 1, seed=33)
    out = ops.fwd(x, [torch.from_numpy(w).cuda() for w in ws])
    got = out[torch.from_numpy(idx).cuda()].float().cpu().numpy()
    del out
    _check(got, orc.forward(xs, ws, round_hidden=True), "sampled rows")


def _check_rows(got, ref, what, tol=2e-4):
    """fp32 tensors: |got - ref| <= tol |ref| + tol max_row |ref|."""
    got = np.asarray(got, np.float64)
    scale = np.abs(ref).max(axis=1, keepdims=True)
    excess = np.abs(got - ref) - (tol * np.abs(ref) + tol * scale)
    assert np.isfinite(got).all() and excess.max() <= 0, f"{what}: worst excess {excess.max():.3g}"


def test_fp32_training_past_2_32_elements():
    # fp32 tensors (bf16 hi/lo split operands): the forward with its stash,
    # then the two-pass backward, whose fp32 dz goes through a 41 GB
    # workspace; the same half-plus-half identity for dW.
    m = M
    rng = np.random.default_rng(34)
    ws = [(rng.standard_normal((DIMS[i], DIMS[i + 1])) / np.sqrt(DIMS[i])).astype(np.float32) for i in range(3)]
    wd = [torch.from_numpy(w).cuda() for w in ws]
    g = torch.Generator(device="cuda").manual_seed(34)
    x = torch.randn((m, DIMS[0]), generator=g, device="cuda", dtype=torch.float32)
    idx = _rows(m)
    ti = torch.from_numpy(idx).cuda()
    xs = x[ti].cpu().numpy()
    out, hs = ops.fwd(x, wd, stash=True)
    ref, ref_h = orc.forward(xs, ws, dtype=np.float64, return_hidden=True)
    _check_rows(out[ti].cpu().numpy(), ref, "sampled rows")
    for i, h in enumerate(hs):
        _check_rows(h[ti].cpu().numpy(), ref_h[i], f"stash h{i + 1}")
    del out
    dout = torch.randn((1, DIMS[-1]), generator=g, device="cuda", dtype=torch.float32).expand(m, DIMS[-1])
    dw = [torch.empty((DIMS[i], DIMS[i + 1]), device="cuda") for i in range(3)]
    ops.bwd(x, wd, hs, dout, dw, accumulate=False)
    half = m // 2
    dwa = [torch.empty_like(d) for d in dw]
    dwb = [torch.empty_like(d) for d in dw]
    ops.bwd(x[:half], wd, [h[:half] for h in hs], dout[:half], dwa, accumulate=False)
    ops.bwd(x[half:], wd, [h[half:] for h in hs], dout[half:], dwb, accumulate=False)
    _check_dw(dw, dwa, dwb, hs[-1], dout[0])
    del x, hs
    torch.cuda.empty_cache()


def test_wide_training_past_2_32_elements(batch):
    # Hidden width 256, 16-bit tensors: the streamed-weight training forward
    # (82 GB of fp32 stash) and the two-pass backward with 16-bit dz through
    # the workspace, whose weight-gradient chunks run ~770 K rows each here.
    x, _, _, idx, xs = batch
    dims = (128, 256, 256, 128)
    _, ws = orc.make_inputs(dims, 1, seed=35)
    wd = [torch.from_numpy(w).cuda() for w in ws]
    ti = torch.from_numpy(idx).cuda()
    out, hs = ops.fwd(x, wd, stash=True)
    ref, ref_h = orc.forward(xs, ws, round_hidden=True, return_hidden=True)
    _check(out[ti].float().cpu().numpy(), ref, "sampled rows")
    for i, h in enumerate(hs):
        _check(h[ti].cpu().numpy(), ref_h[i], f"stash h{i + 1}")
    del out
    g = torch.Generator(device="cuda").manual_seed(36)
    dout = torch.randn((1, dims[-1]), generator=g, device="cuda", dtype=torch.float16).expand(M, dims[-1])
    dw = [torch.empty((dims[i], dims[i + 1]), device="cuda") for i in range(3)]
    ops.bwd(x, wd, hs, dout, dw, accumulate=False)
    half = M // 2
    dwa = [torch.empty_like(d) for d in dw]
    dwb = [torch.empty_like(d) for d in dw]
    ops.bwd(x[:half], wd, [h[:half] for h in hs], dout[:half], dwa, accumulate=False)
    ops.bwd(x[half:], wd, [h[half:] for h in hs], dout[half:], dwb, accumulate=False)
    _check_dw(dw, dwa, dwb, hs[-1], dout[0])
    del hs
    torch.cuda.empty_cache()


def test_recompute_and_five_layers_past_2_32_elements(batch):
    # The 3-layer backward that recomputes h2 instead of reading it (what
    # the modules run from 2^18 rows) against the stashing one, and the
    # 5-layer training step, whose backward hands dz between its two
    # launches through the workspace (10 GB here).
    x, wd, ws, idx, xs = batch
    g = torch.Generator(device="cuda").manual_seed(37)
    dout = torch.randn((1, DIMS[-1]), generator=g, device="cuda", dtype=torch.float16).expand(M, DIMS[-1])
    _, hs = ops.fwd(x, wd, stash=True)
    dw = [torch.empty((DIMS[i], DIMS[i + 1]), device="cuda") for i in range(3)]
    ops.bwd(x, wd, hs, dout, dw, accumulate=False)
    del hs
    _, hr = ops.fwd(x, wd, stash=True, recompute=True)
    assert hr[-1] is None
    dwr = [torch.empty_like(d) for d in dw]
    ops.bwd(x, wd, hr, dout, dwr, accumulate=False)
    del hr
    for i in range(3):
        rel = ((dwr[i].double() - dw[i].double()).norm() / dw[i].double().norm()).item()
        print(f"recompute dW{i + 1}: |recompute - stash| / |stash| = {rel:.3g}")
        assert rel < 1e-3, (i, rel)

    dims5 = (128,) * 6
    _, ws5 = orc.make_inputs(dims5, 1, seed=38)
    wd5 = [torch.from_numpy(w).cuda() for w in ws5]
    out, hs = ops.fwd(x, wd5, stash=True)
    ti = torch.from_numpy(idx).cuda()
    ref, ref_h = orc.forward(xs, ws5, round_hidden=True, return_hidden=True)
    _check(out[ti].float().cpu().numpy(), ref, "5 layers, sampled rows")
    for i, h in enumerate(hs):
        _check(h[ti].cpu().numpy(), ref_h[i], f"5 layers, stash h{i + 1}")
    del out
    dw5 = [torch.empty((128, 128), device="cuda") for _ in range(5)]
    ops.bwd(x, wd5, hs, dout, dw5, accumulate=False)
    half = M // 2
    dwa = [torch.empty_like(d) for d in dw5]
    dwb = [torch.empty_like(d) for d in dw5]
    ops.bwd(x[:half], wd5, [h[:half] for h in hs], dout[:half], dwa, accumulate=False)
    ops.bwd(x[half:], wd5, [h[half:] for h in hs], dout[half:], dwb, accumulate=False)
    _check_dw(dw5, dwa, dwb, hs[-1], dout[0])
    del hs
    torch.cuda.empty_cache()
