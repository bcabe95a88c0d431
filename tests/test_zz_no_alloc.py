"""``mlpmk_bwd_noalloc`` (the backward with the library's own scratch array in
place of a caller workspace) through the C ABI, against ``mlpmk_bwd_ws`` on
the same inputs and against the CPU oracle.

Two calls in a row share the device's scratch array, the second with a
smaller batch; both must match the workspace entry point bit for bit (with
grids of 64+ workgroups both sum the partials in one fixed order) and the
oracle to the weight-gradient tolerance of the other backward tests.  A
shape whose workspace exceeds the array is rejected before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

from mlpmk import _lib, ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu


def _ptrs(ts):
    return _lib.ptr_array([t.data_ptr() if t is not None else None for t in ts])


def _call(entry, dims, x, ws, hs, dout, dws, dx, workspace=None):
    lib = _lib.get()
    pd, _k1 = _lib.int_array(dims)
    pw, _k2 = _ptrs(ws)
    ph, _k3 = _ptrs(hs)
    pdw, _k4 = _ptrs(dws)
    stream = torch.cuda.current_stream().cuda_stream
    args = [len(dims) - 1, pd, _lib.DTYPE_F16, x.data_ptr(), pw, ph, dout.data_ptr(), 0,
            dx.data_ptr() if dx is not None else None, pdw]
    if entry == "ws":
        args += [workspace.data_ptr(), workspace.numel()]
        rc = lib.mlpmk_bwd_ws(*args, int(x.shape[0]), stream)
    else:
        rc = lib.mlpmk_bwd_noalloc(*args, int(x.shape[0]), stream)
    return rc, lib.mlpmk_last_error().decode()


def _case(dims, m, seed, with_dx, recompute=False):
    x, ws = orc.make_inputs(dims, m, seed=seed)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out, hs = ops.fwd(xd, wd, stash=True, recompute=recompute)
    dout = torch.ones((1, dims[-1]), dtype=torch.float16, device="cuda")  # loss = out.sum(): broadcast row
    return x, ws, xd, wd, hs, dout


def _grads(entry, dims, xd, wd, hs, dout, with_dx):
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
    dx = torch.empty_like(xd) if with_dx else None
    ws_t = None
    if entry == "ws":
        nbytes = ops.bwd_workspace_bytes(dims, int(xd.shape[0]), with_dx)
        ws_t = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
    rc, err = _call(entry, dims, xd, wd, hs, dout, dws, dx, ws_t)
    assert rc == 0, err
    torch.cuda.synchronize()
    return dws, dx


def _check_oracle(dims, x, ws, hs, dws, dx, with_dx):
    m = x.shape[0]
    hidden = [h.cpu().numpy() for h in hs if h is not None]
    if len(hidden) < len(dims) - 2:  # recompute mode: h_{L-1} from the oracle
        hidden = orc.forward(x, ws, return_hidden=True)[1]
    rdws, rdx = orc.backward(x, ws, hidden, np.ones((m, dims[-1]), np.float32), need_dx=with_dx)
    for i, (g, r) in enumerate(zip(dws, rdws)):
        g = g.cpu().numpy().astype(np.float64)
        scale = np.abs(r).max()
        worst = np.max(np.abs(g - r) - (2e-2 * np.abs(r) + 2e-3 * scale))
        frob = np.linalg.norm(g - r) / np.linalg.norm(r)
        assert worst <= 0 and frob < 1e-2, f"dW{i + 1}: worst excess {worst:.3g}, rel frob {frob:.3g}"
    if with_dx:
        ok, err, _ = orc.allclose_report(dx.float().cpu().numpy(), rdx, 1e-2, 1e-2)
        assert ok, f"dx: {err}"


# (dims, first M, second (smaller) M, dx, recompute): every case runs the
# partial-sum path (64+ workgroups), which is where the workspace is used.
CASES = [
    ((128, 128, 128, 128), 131072, 16384, False, False),
    ((128, 128, 128, 128), 131072, 16384, True, False),
    ((128, 128, 128, 128), 131072, 16384, False, True),
    ((128,) * 6, 65536, 32768, True, False),
    ((32, 64, 64, 16), 262144, 65536, True, False),
]


@pytest.mark.parametrize("dims,m1,m2,with_dx,recompute", CASES)
def test_noalloc_matches_workspace_entry_on_two_calls(dims, m1, m2, with_dx, recompute):
    assert m2 < m1
    for call, m in enumerate((m1, m2)):
        x, ws, xd, wd, hs, dout = _case(dims, m, seed=10 + call, with_dx=with_dx, recompute=recompute)
        got_dws, got_dx = _grads("noalloc", dims, xd, wd, hs, dout, with_dx)
        ref_dws, ref_dx = _grads("ws", dims, xd, wd, hs, dout, with_dx)
        for i, (a, b) in enumerate(zip(got_dws, ref_dws)):
            assert torch.equal(a, b), f"call {call} (M={m}): dW{i + 1} differs from mlpmk_bwd_ws"
        if with_dx:
            assert torch.equal(got_dx, ref_dx), f"call {call} (M={m}): dx differs from mlpmk_bwd_ws"
        _check_oracle(dims, x, ws, hs, got_dws, got_dx, with_dx)


def test_noalloc_rejects_shapes_beyond_its_scratch():
    dims = (128,) * 6
    m = 262144  # dz hand-over alone is 64 MiB
    need = ops.bwd_workspace_bytes(dims, m, True)
    assert need > (64 << 20)
    x, ws, xd, wd, hs, dout = _case(dims, m, seed=3, with_dx=True)
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(5)]
    dx = torch.zeros_like(xd)
    rc, err = _call("noalloc", dims, xd, wd, hs, dout, dws, dx)
    assert rc == 2 and "scratch" in err, (rc, err)  # MLPMK_ERR_UNSUPPORTED_SHAPE, nothing launched
    torch.cuda.synchronize()
    assert all(int(torch.count_nonzero(d)) == 0 for d in dws) and int(torch.count_nonzero(dx)) == 0
