"""fp32 tensors through the forward (``mlpmk_fwd`` with MLPMK_DTYPE_F32 and the
drop-in ``kernel._fused_mlp_fwd``): the reference's launcher passes fp32
``x`` on (/root/reference/kernel.py:130-138) and its kernels take fp32
tensors through INPUT_DTYPE (/root/reference/mlp_fused.md:159-166), where
``tl.dot`` rounds the operands to TF32.  Here x, the scaled weights and the
hidden activations are rounded to fp16 MFMA operands (TF32's 10-bit
mantissa), accumulation and softplus are fp32, and ``out`` is written in
fp32 from the accumulators.

Checks: against the exact fp32 oracle at the north_star's atol = rtol = 1e-2;
against the oracle on fp16-rounded x, W and hidden activations at 2e-3; bit
for bit against the fp16 kernel (whose output is the same accumulator
rounded to fp16) on fp16-representable inputs; outputs that are not fp16
values (the fp32 store path); the stash; the exact re-run past u >= 128.
"""
import numpy as np
import pytest
import torch

import kernel
from mlpmk import ops
from oracle import mlp_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-2

SHAPES = [
    ((128, 128, 128, 128), 4096),
    ((128, 128, 128, 128), 131072),
    ((128,) * 6, 16384),
    ((32, 64, 64, 16), 4096),
    ((64, 96, 48, 10), 3001),        # runtime widths, ragged M, output width not a multiple of 4
    ((48, 128, 32), 1000),           # 2 layers
    ((128, 112, 96, 80, 3), 777),    # 4 layers
    ((16, 32, 48, 64, 80, 128), 257),  # 5 layers, runtime widths
]


def _inputs(dims, m, seed):
    """fp32 x and weights with full fp32 mantissas (not fp16 values)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, dims[0])).astype(np.float32)
    ws = [(rng.standard_normal((dims[i], dims[i + 1])) / np.sqrt(dims[i])).astype(np.float32)
          for i in range(len(dims) - 1)]
    return x, ws


def _run(x, ws, stash=False):
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    return ops.fwd(xd, wd, stash=stash)


def _scaled16(ws):
    """The fp16 operands the kernels stage: W_1 * log2(e), W_L * ln(2), rounded
    once from fp32 (and undone in float64, so the oracle sees the same values
    the MFMA multiplies, in natural units)."""
    L = len(ws)
    out = []
    for i, w in enumerate(ws):
        sc = (np.float32(1.4426950408889634) if i == 0 else np.float32(1)) * (np.float32(0.6931471805599453) if i == L - 1 else np.float32(1))
        w16 = (w.astype(np.float32) * sc).astype(np.float16).astype(np.float64)
        out.append(w16 / float(sc))
    return out


@pytest.mark.parametrize("dims,m", SHAPES)
def test_fp32_forward_matches_oracle(dims, m):
    x, ws = _inputs(dims, m, seed=len(dims) * 1000 + m)
    out = _run(x, ws)
    assert out.dtype == torch.float32 and tuple(out.shape) == (m, dims[-1])
    got = out.cpu().numpy()
    ok, err, _ = orc.allclose_report(got, orc.forward(x, ws), TOL, TOL)
    assert ok, f"vs exact fp32 oracle: max|err| {err}"
    # the operands the kernel claims: fp16 x, fp16 scaled W, fp16 hidden activations
    ref16 = orc.forward(x.astype(np.float16), _scaled16(ws), round_hidden=True, dtype=np.float64)
    ok, err, _ = orc.allclose_report(got, ref16, 2e-3, 2e-3)
    assert ok, f"vs oracle on fp16 operands: max|err| {err}"
    # written from the fp32 accumulators, not rounded to fp16
    assert np.mean(got != got.astype(np.float16).astype(np.float32)) > 0.5


@pytest.mark.parametrize("dims,m", [((128, 128, 128, 128), 4096), ((128, 128, 128, 128), 1048576),
                                    ((128,) * 6, 65536), ((32, 64, 64, 16), 262144), ((64, 96, 48, 10), 3001)])
def test_fp32_kernel_is_the_fp16_kernel_before_the_output_rounding(dims, m):
    # On fp16-representable inputs both kernels compute the same accumulators
    # (same staged weights, operands and K order); the fp16 kernel rounds them
    # to fp16 (RNE), which is what rounding the fp32 output gives.
    x, ws = orc.make_inputs(dims, m, seed=5)
    x16 = torch.from_numpy(x).cuda()
    w16 = [torch.from_numpy(w).cuda() for w in ws]
    out16 = ops.fwd(x16, w16)
    out32 = ops.fwd(x16.float(), [w.float() for w in w16])
    assert torch.equal(out32.half(), out16)


def test_fp32_stash_matches_oracle_hidden():
    dims, m = (128, 128, 128, 128), 8192
    x, ws = _inputs(dims, m, seed=11)
    out, hs = _run(x, ws, stash=True)
    ref, hidden = orc.forward(x, ws, return_hidden=True)
    ok, err, _ = orc.allclose_report(out.cpu().numpy(), ref, TOL, TOL)
    assert ok, err
    for i, (h, r) in enumerate(zip(hs, hidden)):
        ok, err, _ = orc.allclose_report(h.cpu().numpy(), r, TOL, TOL)
        assert ok, f"h{i + 1}: {err}"
    # the inference kernel gives the same output bits as the training one
    assert torch.equal(_run(x, ws), out)


def test_fp32_large_preactivations_take_the_exact_rerun():
    # Rows whose pre-activations reach z > 88.7 (2^u overflows fp32) re-run in
    # the exact form: softplus(z) = z there, as the reference's threshold
    # gives.  On fp16-representable inputs the fp32 kernel is the fp16 one
    # before the output rounding (whose exact path test_fwd_gpu.py checks),
    # bit for bit; against the oracle, rows scaled by 400 carry intermediate
    # terms of several hundred that cancel in some outputs, so each row's
    # atol is 1e-2 of the row's largest |out| (fp16 operands: 2^-11 relative).
    dims, m = (128, 128, 128, 128), 4096
    x, ws = orc.make_inputs(dims, m, seed=3)
    big = np.arange(m) % 97 == 0
    x[big] = (x[big].astype(np.float32) * 400.0).astype(np.float16)  # |x| up to ~2000
    x16 = torch.from_numpy(x).cuda()
    w16 = [torch.from_numpy(w).cuda() for w in ws]
    out16 = ops.fwd(x16, w16)
    out32 = ops.fwd(x16.float(), [w.float() for w in w16])
    assert torch.equal(out32.half(), out16)
    got = out32.cpu().numpy().astype(np.float64)
    ref = orc.forward(x, ws).astype(np.float64)
    assert np.isfinite(got).all()
    assert np.abs(ref[big]).max() > 100.0  # the scaled rows went through large activations
    row_scale = np.abs(ref).max(axis=1, keepdims=True)
    err = np.abs(got - ref)
    assert np.all(err <= TOL + TOL * np.abs(ref) + TOL * row_scale * big[:, None]), float(err.max())
    ok, e2, _ = orc.allclose_report(got[~big], ref[~big], TOL, TOL)
    assert ok, e2


@pytest.mark.parametrize("xview,wview", [("contiguous", "contiguous"), ("transposed", "sliced")])
def test_fp32_launcher_matches_model_and_oracle(xview, wview):
    dims, m = (128, 128, 128, 128), 4096
    x, ws = _inputs(dims, m, seed=21)
    xd = torch.from_numpy(x).cuda()
    wd = [torch.from_numpy(w).cuda() for w in ws]
    if xview == "transposed":
        xd = xd.t().contiguous().t()  # same values, column-major storage
    if wview == "sliced":
        wd = [torch.cat([w, w], dim=1)[:, : w.shape[1]] for w in wd]  # non-contiguous views
    out = kernel._fused_mlp_fwd(xd, *wd)
    assert out.dtype == torch.float32
    ok, err, _ = orc.allclose_report(out.cpu().numpy(), orc.forward(x, ws), TOL, TOL)
    assert ok, err
    eager = kernel.Model()(xd, *wd)  # the reference's eager fp32 model on the GPU
    ok, err, _ = orc.allclose_report(out.cpu().numpy(), eager.cpu().numpy(), TOL, TOL)
    assert ok, err
    assert torch.equal(kernel.ModelNew()(xd, *wd), out)


def test_fp32_small_and_empty_batches():
    dims = (128, 128, 128, 128)
    for m in (0, 1, 31, 33, 255):
        x, ws = _inputs(dims, m, seed=m)
        out = _run(x, ws)
        assert tuple(out.shape) == (m, 128)
        if m:
            ok, err, _ = orc.allclose_report(out.cpu().numpy(), orc.forward(x, ws), TOL, TOL)
            assert ok, (m, err)


def test_mixed_dtypes_are_rejected():
    x = torch.zeros((64, 128), device="cuda", dtype=torch.float32)
    ws = [torch.zeros((128, 128), device="cuda", dtype=torch.float16) for _ in range(3)]
    with pytest.raises(TypeError):
        ops.fwd(x, ws)
