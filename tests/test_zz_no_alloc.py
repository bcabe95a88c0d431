"""``mlpmk_bwd_noalloc`` (the backward with the library's own scratch array in
place of a caller workspace) through the C ABI, against ``mlpmk_bwd_ws`` on
the same inputs and against the CPU oracle.

Two calls in a row share the device's scratch array, the second with a
smaller batch; both must match the workspace entry point -- bit for bit
where the one-pass megakernel runs (its partials are summed in one fixed
order), to fp32 summation order where the two-pass backward does (up to
16,384 rows: fp32 atomics) -- and the oracle to the weight-gradient
tolerance of the other backward tests.  A
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


def _call(entry, dims, x, ws, hs, dout, dws, dx, workspace=None, dtype=_lib.DTYPE_F16):
    lib = _lib.get()
    pd, _k1 = _lib.int_array(dims)
    pw, _k2 = _ptrs(ws)
    ph, _k3 = _ptrs(hs)
    pdw, _k4 = _ptrs(dws)
    stream = torch.cuda.current_stream().cuda_stream
    args = [len(dims) - 1, pd, dtype, x.data_ptr(), pw, ph, dout.data_ptr(), 0,
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
            if m > 16384:
                assert torch.equal(a, b), f"call {call} (M={m}): dW{i + 1} differs from mlpmk_bwd_ws"
            else:  # two-pass backward: fp32 atomics, any summation order
                assert torch.allclose(a, b, rtol=1e-5, atol=1e-6 * float(b.abs().max())), f"call {call}: dW{i + 1}"
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


# The 64 MiB claim of mlpmk.h: every 2- and 3-layer network mlpmk_bwd_supported
# accepts needs at most MLPMK_NOALLOC_SCRATCH_BYTES of workspace at any M
# (the weight-gradient partials are one dW copy per workgroup of a grid
# capped at the CU count times the occupancy), fp16 and bf16, with and
# without dx; the 5-layer 128-wide network up to 65,536 rows.
NOALLOC_BYTES = 64 << 20
SWEEP_DIMS = [
    (128, 128, 128, 128), (32, 64, 64, 16), (128, 128, 128), (16, 16, 16), (16, 128, 1),
    (128, 112, 128, 128), (48, 96, 80, 10), (112, 128, 96, 128), (128, 128, 7),
]


@pytest.mark.parametrize("dims", SWEEP_DIMS)
def test_two_and_three_layer_workspace_fits_the_scratch_at_any_batch(dims):
    assert ops.bwd_supported(list(dims))
    for dt in (torch.float16, torch.bfloat16):
        for with_dx in (False, True):
            sizes = [ops.bwd_workspace_bytes(dims, m, with_dx, dtype=dt)
                     for m in (1, 4096, 16384, 65536, 131072, 1 << 20, 1 << 24, (1 << 31) - 1)]
            assert max(sizes) <= NOALLOC_BYTES, (dims, dt, with_dx, sizes)


def test_five_layer_workspace_fits_up_to_65536_rows():
    for with_dx in (False, True):
        assert ops.bwd_workspace_bytes((128,) * 6, 65536, with_dx) <= NOALLOC_BYTES
        assert ops.bwd_workspace_bytes((128,) * 6, 262144, with_dx) > NOALLOC_BYTES


# The first mlpmk_bwd_noalloc call of a process made inside a HIP graph
# capture (the scratch array's address is looked up on that call), then the
# graph replayed with fresh inputs and each replay checked against the
# oracle.  Runs in a child process so that the call really is the first.
_CAPTURE_SCRIPT = r'''
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np, torch
import _mlpmk  # noqa: F401
from mlpmk import _lib, ops
from oracle import mlp_oracle as orc

dims, m = (128, 128, 128, 128), 16384
lib = _lib.get()
x0, ws = orc.make_inputs(dims, m, seed=41)
wd = [torch.from_numpy(w).cuda() for w in ws]
xd = torch.from_numpy(x0).cuda()
hs = [torch.empty((m, 128), dtype=torch.float32, device="cuda") for _ in range(2)]
out = torch.empty((m, 128), dtype=torch.float16, device="cuda")
dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]
dout = torch.ones((1, 128), dtype=torch.float16, device="cuda")
pd, k1 = _lib.int_array(list(dims))
pw, k2 = _lib.ptr_array([w.data_ptr() for w in wd])
ph, k3 = _lib.ptr_array([h.data_ptr() for h in hs])
pg, k4 = _lib.ptr_array([d.data_ptr() for d in dws])
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
ops.fwd_into(xd, wd, out, hs)  # forward kernels loaded outside the capture
torch.cuda.synchronize()
with torch.cuda.graph(g, stream=s):
    for d in dws:
        d.zero_()
    ops.fwd_into(xd, wd, out, hs)
    rc = lib.mlpmk_bwd_noalloc(3, pd, _lib.DTYPE_F16, xd.data_ptr(), pw, ph, dout.data_ptr(), 0, None, pg, m,
                               torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.mlpmk_last_error().decode()
torch.cuda.synchronize()
for rep in range(3):
    x, _ = orc.make_inputs(dims, m, seed=100 + rep)
    xd.copy_(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    _, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True)
    rdws, _ = orc.backward(x, ws, ref_h, np.ones((m, 128), np.float32), need_dx=False)
    for i in range(3):
        got = dws[i].cpu().numpy().astype(np.float64)
        r = rdws[i].astype(np.float64)
        worst = np.max(np.abs(got - r) - (2e-2 * np.abs(r) + 2e-3 * np.abs(r).max()))
        frob = np.linalg.norm(got - r) / np.linalg.norm(r)
        assert worst <= 0 and frob < 1e-2, (rep, i, worst, frob)
print("capture ok")
'''


def test_first_noalloc_call_inside_a_graph_capture():
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, root], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "capture ok" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]


_CODES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


@pytest.mark.parametrize("dims,dt,m1,m2,with_dx", [
    ((128, 256, 256, 128), torch.float16, 16384, 4096, True),  # widths above 128: the two-pass form
    ((128, 128, 128, 128), torch.float32, 32768, 4096, True),  # fp32 tensors: fp32 dz in the scratch
    ((64, 96, 48, 16), torch.bfloat16, 20000, 3000, False),    # bf16, one-pass then two-pass
])
def test_noalloc_other_types_and_widths_on_two_calls(dims, dt, m1, m2, with_dx):
    # The same two-call check for the element types and widths whose
    # backward hands dz through the scratch (two-pass) or sums partials there.
    code = _CODES[dt]
    for call, m in enumerate((m1, m2)):
        x, ws = orc.make_inputs(dims, m, seed=20 + call, elem="bf16" if dt == torch.bfloat16 else "f16")
        xd = torch.from_numpy(x).cuda().to(dt)
        wd = [torch.from_numpy(w).cuda().to(dt) for w in ws]
        _, hs = ops.fwd(xd, wd, stash=True)
        dout = torch.ones((1, dims[-1]), dtype=dt, device="cuda")
        got = []
        for entry in ("noalloc", "ws"):
            dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(len(dims) - 1)]
            dx = torch.empty_like(xd) if with_dx else None
            ws_t = None
            if entry == "ws":
                nbytes = ops.bwd_workspace_bytes(dims, m, with_dx, dtype=dt)
                ws_t = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
            rc, err = _call(entry, dims, xd, wd, hs, dout, dws, dx, ws_t, dtype=code)
            assert rc == 0, f"{entry} call {call}: {err}"
            torch.cuda.synchronize()
            got.append((dws, dx))
        (a_dws, a_dx), (b_dws, b_dx) = got
        for i, (a, b) in enumerate(zip(a_dws, b_dws)):
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-6 * float(b.abs().max())), f"call {call}: dW{i + 1}"
        if with_dx:
            assert torch.equal(a_dx, b_dx), f"call {call}: dx differs from mlpmk_bwd_ws"
        # and the oracle, on the same (16-bit or fp32) values
        ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=dt != torch.float32,
                            elem="bf16" if dt == torch.bfloat16 else "f16")[1]
        rdws, _ = orc.backward(x, ws, ref_h, np.ones((m, dims[-1]), np.float32), need_dx=False)
        k = 2.0 if dt == torch.bfloat16 else 1.0
        for i, (g, r) in enumerate(zip(a_dws, rdws)):
            g = g.cpu().numpy().astype(np.float64)
            scale = np.abs(r).max()
            worst = np.max(np.abs(g - r) - k * (2e-2 * np.abs(r) + 2e-3 * scale))
            frob = np.linalg.norm(g - r) / np.linalg.norm(r)
            assert worst <= 0 and frob < k * 1e-2, f"call {call} dW{i + 1}: worst excess {worst:.3g}, frob {frob:.3g}"
