"""MLPMK_BWD_WRITE_DW: the backward writes dW (=) instead of accumulating
into it (+=).  On every route of the backward -- the two-pass form (whose
data-gradient pass clears dW before the weight-gradient pass adds), the
one-pass megakernel with its partial-sum combine (which then stores), and
the one-pass kernel adding with atomics straight into dW (cleared by a
launch of its own first) -- a dW block pre-filled with NaN must come out
equal to the accumulating call into zeros: bit for bit where the summation
order is fixed (the combine), within fp32 rounding where atomics add in any
order.  dx is the same either way."""
import numpy as np
import pytest
import torch

from mlpmk import ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu

# (dims, M, dtype, workspace, recompute, exact): which route each case takes
# is noted beside it.
CASES = [
    ((128,) * 4, 4096, torch.float16, True, False, False),          # two-pass (dz through the workspace)
    ((128,) * 4, 4096, torch.float32, True, False, False),          # two-pass, fp32 split operands
    ((128, 256, 256, 128), 4096, torch.float16, True, False, False),  # two-pass, widths above 128
    ((128,) * 4, 131072, torch.float16, True, False, True),         # one-pass + combine (fixed order)
    ((128,) * 4, 4096, torch.float16, False, False, False),         # one-pass, atomics into dW (no workspace)
    ((128,) * 4, 4096, torch.float16, True, True, False),           # one-pass recomputing kernel, atomics
    ((128,) * 6, 32768, torch.float16, True, False, True),          # 5 layers: two one-pass launches + combines
    ((64, 96, 48, 10), 3001, torch.float16, True, False, False),    # runtime widths, odd output: one-pass
]


@pytest.mark.parametrize("dims,m,dt,workspace,recompute,exact", CASES)
def test_written_dw_equals_accumulated_into_zeros(dims, m, dt, workspace, recompute, exact):
    x, ws = orc.make_inputs(dims, m, seed=m % 101 + len(dims))
    xd = torch.from_numpy(x).cuda().to(dt)
    wd = [torch.from_numpy(w).cuda().to(dt) for w in ws]
    out, hs = ops.fwd(xd, wd, stash=True, recompute=recompute)
    g = torch.Generator(device="cuda").manual_seed(5)
    dout = torch.randn(out.shape, generator=g, device="cuda").to(dt)
    ref = [torch.zeros(w.shape, dtype=torch.float32, device="cuda") for w in wd]
    dx_ref = torch.empty_like(xd)
    ops.bwd(xd, wd, hs, dout, ref, dx_ref, workspace=workspace)
    got = [torch.full(w.shape, float("nan"), dtype=torch.float32, device="cuda") for w in wd]
    dx = torch.empty_like(xd)
    ops.bwd(xd, wd, hs, dout, got, dx, workspace=workspace, accumulate=False)
    # a second written call on the same blocks must not add to the first
    ops.bwd(xd, wd, hs, dout, got, dx, workspace=workspace, accumulate=False)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(got, ref)):
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert np.isfinite(a).all(), f"dW{i}: NaN left from the pre-fill"
        if exact:
            assert np.array_equal(a, b), f"dW{i}: written and accumulated differ"
        else:
            scale = np.abs(b).max()
            assert np.abs(a - b).max() <= 1e-5 * scale, f"dW{i}: max diff {np.abs(a - b).max():.3g} (scale {scale:.3g})"
    assert torch.equal(dx, dx_ref)
