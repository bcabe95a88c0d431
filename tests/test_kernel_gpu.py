"""The drop-in inference surface of /root/reference/kernel.py on the GPU.

``kernel._fused_mlp_fwd(x, w1, w2, w3)`` (kernel.py:130-156) and ``ModelNew``
(kernel.py:174-180) against the CPU oracle and against the reference's own
eager ``Model`` (kernel.py:163-171) run on the GPU, with the tolerance of
/root/reference/profile.py:92 (atol = rtol = 1e-2).  The reference copies
non-contiguous inputs (kernel.py:132-133); transposed and sliced views of
``x`` and of the weights must give the result of their contiguous copies.
"""
import numpy as np
import pytest
import torch

import kernel
from mlpmk import ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _inputs(m, seed):
    x, ws = orc.make_inputs((128, 128, 128, 128), m, seed=seed)
    return torch.from_numpy(x).cuda(), [torch.from_numpy(w).cuda() for w in ws], x, ws


def _transposed(t):
    """A transposed view holding t's values (stride (1, rows))."""
    return t.t().contiguous().t()


def _sliced(t):
    """A column slice of a wider tensor holding t's values (row stride 2 * cols)."""
    big = torch.zeros((t.shape[0], 2 * t.shape[1]), dtype=t.dtype, device=t.device)
    big[:, 3 : 3 + t.shape[1]] = t
    return big[:, 3 : 3 + t.shape[1]]


def _strided_rows(t):
    """Every other row of a taller tensor (row stride 2 * cols)."""
    big = torch.zeros((2 * t.shape[0], t.shape[1]), dtype=t.dtype, device=t.device)
    big[::2] = t
    return big[::2]


VIEWS = {"contiguous": lambda t: t, "transposed": _transposed, "sliced": _sliced, "strided_rows": _strided_rows}


@pytest.mark.parametrize("m", [256, 4096])  # BASELINE configs[0] (M = 256) and the sweep's largest point
@pytest.mark.parametrize("xview", list(VIEWS))
@pytest.mark.parametrize("wview", ["contiguous", "transposed", "sliced"])
def test_fused_mlp_fwd_matches_oracle_and_eager_model(m, xview, wview):
    xd, wd, x, ws = _inputs(m, seed=0)
    xv = VIEWS[xview](xd)
    wv = [VIEWS[wview](w) for w in wd]
    assert torch.equal(xv, xd) and all(torch.equal(a, b) for a, b in zip(wv, wd))
    if xview != "contiguous":
        assert not xv.is_contiguous()
    if wview != "contiguous":
        assert not any(w.is_contiguous() for w in wv)
    out = kernel._fused_mlp_fwd(xv, *wv)
    assert out.shape == (m, 128) and out.dtype == torch.float16 and out.is_contiguous()
    # the views change nothing: same bits as the library on contiguous copies
    assert torch.equal(out, ops.fwd(xd, wd))
    got = out.float().cpu().numpy()
    ok, err, _ = orc.allclose_report(got, orc.forward(x, ws), TOL, TOL)
    assert ok, f"vs oracle: max|err| {err}"
    # the reference's eager Model on the GPU (fp16 rocBLAS products, z rounded
    # to fp16 before the softplus); contiguous operands for the products
    eager = kernel.Model()(xd, *wd).float().cpu().numpy()
    ok, err, _ = orc.allclose_report(got, eager, TOL, TOL)
    assert ok, f"vs eager Model: max|err| {err}"


@pytest.mark.parametrize("m", [256, 4096])
def test_model_new_matches_model(m):
    xd, wd, x, ws = _inputs(m, seed=1)
    new = kernel.ModelNew()(_transposed(xd), *[_sliced(w) for w in wd])
    ref = kernel.Model()(xd, *wd)
    torch.testing.assert_close(new, ref, atol=TOL, rtol=TOL)
    ok, err, _ = orc.allclose_report(new.float().cpu().numpy(), orc.forward(x, ws), TOL, TOL)
    assert ok, f"ModelNew vs oracle: max|err| {err}"


def test_launcher_runs_on_the_current_stream_without_sync():
    xd, wd, x, ws = _inputs(4096, seed=2)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = kernel._fused_mlp_fwd(xd, *wd)
    s.synchronize()
    ok, err, _ = orc.allclose_report(out.float().cpu().numpy(), orc.forward(x, ws), TOL, TOL)
    assert ok, err


_MIRROR_DIMS = [(128,) * 4, (32, 64, 64, 16), (64, 64, 64, 64), (128, 128, 128, 10), (64, 128, 32, 16),
                (128, 256, 256, 128)]


# (fp32 tensors run widths up to 128: no fp32 case for the wide network)
@pytest.mark.parametrize("dims,fp32", [(d, f) for d in _MIRROR_DIMS for f in (False, True) if not (f and max(d) > 128)])
def test_pick_config_mirror_matches_the_library_launch(dims, fp32):
    # The Python mirror of the launch policy (used without a device) against
    # the library's own answer from the code path that launches
    # (mlpmk_fwd_launch_info), at the sizes where the policy switches; fp16
    # and fp32 tensors.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    dt = torch.float32 if fp32 else torch.float16
    for m in (1, 64, 32 * cus, 32 * cus + 1, 64 * cus, 64 * cus + 1, 128 * cus, 128 * cus + 1, 256 * cus,
              256 * cus + 1, 512 * cus + 1, 1048576):
        info = ops.fwd_launch_info(dims, m, dtype=dt)
        assert kernel._mirror_policy(m, dims, cus, fp32=fp32) == (info["rows_per_block"], info["waves"]), (dims, m, info)
        assert kernel._pick_config(m, *dims, fp32=fp32)[::5] == (info["rows_per_block"], info["waves"])
        nblk = -(-m // info["rows_per_block"])
        per_wg = 1 if info["kernel"] == "feature_split" else info["waves"]
        assert info["grid"] == min(-(-nblk // per_wg), cus * info["wgs_per_cu"]), (dims, m, info)


def test_fwd_launch_info_edge_cases():
    assert ops.fwd_launch_info((128,) * 4, 0)["kernel"] == "none"
    with pytest.raises(ops.MlpmkError):
        ops.fwd_launch_info((128, 272, 128, 128), 4096)  # no kernel above 256 features
