"""A seeded sweep of network shapes through the C ABI on the GPU: forward
(training forward with the fp32 stash) and fused backward against the CPU
oracle, for networks drawn at random from everything the fused kernels take
-- 2..5 layers, input and hidden widths multiples of 16 up to 256, any
output width up to 256, ragged batches, fp16 and bf16 tensors, dense or
broadcast dL/dout, with or without dx (the few shapes without a fused
backward -- widths above 128 with an output width not a multiple of 8 --
through the library-GEMM backward that trains them).  The fixed cases of
the other files pin each kernel family; this sweep covers their
combinations (a 5-layer network with one 256-wide layer, a 2-layer network
with a 1-wide output, ...).
The reference's kernel takes any tile-multiple width as constexpr tile loops
(/root/reference/kernel.py:60-63,86-87,121-123) and its modules take D, H,
out_features (/root/reference/README.md:62,68).

A second sweep draws fp32-tensor networks (widths up to 128, the split-
operand kernels).

Tolerances are those of the per-dtype files: outputs at atol = rtol = 1e-2
(fp16) and 3e-2 (bf16); weight gradients per entry within 2e-2 |ref| + 2e-3
max|ref| and relative Frobenius 1e-2 (fp16), 4e-2 |ref| + (L + 1) 1e-3
max|ref| and 2e-2 (bf16); dx as the outputs.
"""
import numpy as np
import pytest
import torch

from mlpmk import ops
from oracle import mlp_oracle as orc
from test_bf16_gpu import check_dw_bf16
from test_bwd_gpu import check_dw

pytestmark = pytest.mark.gpu


def _draw_cases(n, seed=2026):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        L = int(rng.integers(2, 6))
        wide = rng.random() < 0.35  # some layer above 128: the streamed-weight forward, two-pass backward
        top = 256 if wide else 128
        dims = [16 * int(rng.integers(1, top // 16 + 1)) for _ in range(L)]
        dims.append(int(rng.integers(1, top + 1)) if rng.random() < 0.5 else 8 * int(rng.integers(1, top // 8 + 1)))
        m = int(rng.choice([1, 31, 33, 777, 4099, 20000, 65536 + 3]))
        elem = "bf16" if rng.random() < 0.4 else "f16"
        dout_mode = "ones" if rng.random() < 0.5 else "dense"
        with_dx = bool(rng.random() < 0.5)
        if not ops.fwd_supported(dims):
            continue
        cases.append((tuple(dims), m, elem, dout_mode, with_dx))
    return cases


CASES = _draw_cases(64)


def _ids(case):
    dims, m, elem, dout_mode, with_dx = case
    return f"{'-'.join(map(str, dims))}_M{m}_{elem}_{dout_mode}{'_dx' if with_dx else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_random_shape_train_matches_oracle(case):
    dims, m, elem, dout_mode, with_dx = case
    L = len(dims) - 1
    tdt = torch.bfloat16 if elem == "bf16" else torch.float16
    tol = 3e-2 if elem == "bf16" else 1e-2
    seed = sum(dims) * 7 + m
    x, ws = orc.make_inputs(dims, m, seed=seed % 1000, elem=elem)
    xd = torch.from_numpy(x).cuda().to(tdt)
    wd = [torch.from_numpy(w).cuda().to(tdt) for w in ws]
    print(f"case {_ids(case)}", flush=True)

    out, hs = ops.fwd(xd, wd, stash=True)
    assert out.dtype == tdt and out.shape == (m, dims[-1])
    ref, ref_h = orc.forward(x, ws, return_hidden=True, round_hidden=True, elem=elem)
    ok, err, excess = orc.allclose_report(out.float().cpu().numpy(), ref, tol, tol)
    assert ok, f"out: max|err|={err:.4g}, worst excess {excess:.4g}"
    assert torch.equal(out, ops.fwd(xd, wd)), "inference and training forward differ"

    fused = ops.bwd_supported(list(dims), tdt)
    if dout_mode == "ones":
        dout_np = np.ones((m, dims[-1]), np.float32)
        dout = torch.ones((1, dims[-1]), dtype=tdt, device="cuda").expand(m, dims[-1])
    else:
        dout_np = np.random.default_rng(seed + 1).standard_normal((m, dims[-1])).astype(np.float32)
        dout_np = orc.round_elem(dout_np, elem)
        dout = torch.from_numpy(dout_np).cuda().to(tdt)
    dws = [torch.zeros((dims[i], dims[i + 1]), dtype=torch.float32, device="cuda") for i in range(L)]
    dx = torch.empty_like(xd) if with_dx else None
    if fused:
        ops.bwd(xd, wd, hs, dout, dws, dx, accumulate=False)
    else:  # widths above 128 with an output width not a multiple of 8: the library-GEMM backward
        from mlpmk import fallback

        fallback.bwd(xd, wd, hs, dout, dws, dx)
    rdws, rdx = orc.backward(x, ws, ref_h, dout_np, need_dx=with_dx)
    for i in range(L):
        got = dws[i].cpu().numpy()
        if elem == "bf16":
            check_dw_bf16(got, rdws[i], f"dW{i + 1}", L)
        else:
            check_dw(got, rdws[i], f"dW{i + 1}")
    if with_dx:
        ok, err, excess = orc.allclose_report(dx.float().cpu().numpy(), rdx, tol, tol)
        assert ok, f"dx: max|err|={err:.4g}, worst excess {excess:.4g}"


def _draw_cases_f32(n, seed=2027):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        L = int(rng.integers(2, 6))
        dims = [16 * int(rng.integers(1, 9)) for _ in range(L)]
        dims.append(int(rng.integers(1, 129)) if rng.random() < 0.4 else 8 * int(rng.integers(1, 17)))
        m = int(rng.choice([1, 33, 777, 4099, 20000]))
        if ops.fwd_supported(dims, torch.float32):
            cases.append((tuple(dims), m))
    return cases


CASES_F32 = _draw_cases_f32(24)


@pytest.mark.parametrize("dims,m", CASES_F32, ids=[f"{'-'.join(map(str, d))}_M{m}" for d, m in CASES_F32])
def test_random_shape_fp32_matches_oracle(dims, m):
    # fp32 tensors (bf16 hi/lo split operands) at the tolerances of
    # test_fp32_gpu.py: outputs and dx within 2e-4 of their row's scale,
    # weight gradients within 1e-3 |ref| + 1e-4 max|ref|, relative Frobenius
    # 5e-4, against the oracle in float64.
    from test_fp32_gpu import _check_dw32, _check_rows, _inputs, _train32

    print(f"case fp32 {dims} M={m}", flush=True)
    x, ws = _inputs(dims, m, seed=sum(dims) + m)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    out = ops.fwd(xd, wd)
    assert out.dtype == torch.float32 and out.shape == (m, dims[-1])
    _check_rows(out.cpu().numpy(), orc.forward(x, ws, dtype=np.float64), "out")
    if not ops.bwd_supported(list(dims), torch.float32):
        return  # fp32 output widths not a multiple of 8: the library-GEMM backward (test_fp32_gpu.py)
    dws, dx, rdws, rdx = _train32(dims, m, seed=sum(dims) + m, dout_mode="dense", with_dx=True)
    for i in range(len(dims) - 1):
        _check_dw32(dws[i].cpu().numpy(), rdws[i], f"dW{i + 1}")
    _check_rows(dx.cpu().numpy(), rdx, "dx")
