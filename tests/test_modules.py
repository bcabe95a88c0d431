"""Host-side plumbing of the drop-in modules (no GPU needed): parameter
layout and initialisation, state_dict round trip, weight-norm views, the
broadcast handling of ``loss = out.sum()`` gradients, and that the product
path refuses CPU tensors instead of computing anything on the CPU."""
import math

import pytest
import torch

import fused_mlp
import fused_mlp5
import kernel
from mlpmk.autograd import _as_row_broadcast, _layout, _split


def test_parameter_layout_and_init():
    torch.manual_seed(0)
    m = fused_mlp.FusedMLPSoftplus(D=32, H=64, out_features=16)
    assert m.dims == (32, 64, 64, 16)
    shapes = [tuple(p.shape) for p in m.parameters()]
    assert shapes == [(32, 64), (64, 64), (64, 16)]  # [in, out], as kernel.py:105,109,113 index W
    big = fused_mlp.FusedMLPSoftplus()
    for p, fan_in in zip(big.weights, (128, 128, 128)):
        assert abs(float(p.std()) - 1 / math.sqrt(fan_in)) < 0.01
    assert fused_mlp5.FusedMLP5Softplus().dims == (128,) * 6


def test_state_dict_round_trip():
    a = fused_mlp.FusedMLPSoftplusWN()
    b = fused_mlp.FusedMLPSoftplusWN()
    b.load_state_dict(a.state_dict())
    assert set(a.state_dict()) == {"v_all", "g_all"}
    assert torch.equal(a.v_all, b.v_all) and torch.equal(a.g_all, b.g_all)


def test_weight_norm_blocks_are_contiguous_views():
    m = fused_mlp.FusedMLPSoftplusWN(D=32, H=64, out_features=16)
    assert m.v_all.numel() == 32 * 64 + 64 * 64 + 64 * 16
    assert m.g_all.numel() == 64 + 64 + 16
    assert torch.all(m.g_all == 1)
    v1 = m.v(1)
    assert v1.shape == (64, 64) and v1.data_ptr() == m.v_all.data_ptr() + 32 * 64 * 4
    assert m.g(2).shape == (16,) and m.g(2).data_ptr() == m.g_all.data_ptr() + 128 * 4
    flat = torch.arange(10.0)
    parts = _split(flat, (1, 2, 4))
    assert [tuple(p.shape) for p in parts] == [(1, 2), (2, 4)] and parts[1][1, 3] == 9
    # The autograd Functions launch on element offsets into the flat blocks
    # (no per-layer views): they must be where _split's views start.
    nw, ng, woff = _layout((32, 64, 64, 16))
    views = _split(m.v_all.detach(), m.dims)
    assert nw == m.v_all.numel() and ng == m.g_all.numel()
    assert [m.v_all.data_ptr() + 4 * o for o in woff] == [v.data_ptr() for v in views]


def test_sum_gradient_stays_one_element():
    # What out.sum() hands back stays as it is (the kernels read its one
    # element, MLPMK_DOUT_SCALAR); ops._dout_rows tags it so.
    from mlpmk import ops

    g = torch.ones((), dtype=torch.float16).expand(5, 7)
    assert g.stride() == (0, 0)
    r = _as_row_broadcast(g)
    assert r is g
    d, st = ops._dout_rows(r, 5, 7, torch.float16, r.device)
    assert d is r and st == ops.DOUT_SCALAR
    assert ops.DOUT_SCALAR == -1
    row = torch.randn(1, 7).half().expand(5, 7)
    assert _as_row_broadcast(row).stride() == (0, 1)
    dense = torch.randn(7, 5).half().t()
    assert _as_row_broadcast(dense).is_contiguous()


def test_misaligned_dout_rows_are_copied():
    # The gradient of a column slice of torch.cat([a, out, b], 1): unit
    # column stride, a row stride that is a multiple of 8, but a first
    # element 4 elements (8 bytes) past a 16-byte boundary.  The library
    # reads dout rows from 16-byte boundaries, so _dout_rows copies it into
    # aligned rows instead of passing it through.
    from mlpmk import ops

    base = torch.randn(6, 136).half()
    assert base.data_ptr() % 16 == 0
    g = base[:, 4:132]
    assert g.stride() == (136, 1) and g.data_ptr() % 16 == 8
    d, st = ops._dout_rows(g, 6, 128, torch.float16, g.device)
    assert d.data_ptr() % 16 == 0 and st % 8 == 0 and st >= 128
    assert torch.equal(d[:, :128], g)
    aligned = base[:, 8:136]
    d2, st2 = ops._dout_rows(aligned, 6, 128, torch.float16, aligned.device)
    assert d2 is aligned and st2 == 136  # an aligned slice goes through as is


def test_product_path_refuses_cpu_tensors():
    m = fused_mlp.FusedMLPSoftplus().half()
    with pytest.raises(ValueError, match="GPU"):
        m(torch.randn(4, 128).half())
    x = torch.randn(4, 128).half()
    ws = [torch.randn(128, 128).half() for _ in range(3)]
    with pytest.raises(ValueError, match="GPU"):
        kernel._fused_mlp_fwd(x, *ws)
    with pytest.raises(ValueError, match="GPU"):
        fused_mlp.FusedMLPSoftplusWN()(torch.randn(4, 128).half())
    # The eager reference model of kernel.py stays available and runs anywhere.
    ref = kernel.Model()(x.float(), *[w.float() for w in ws])
    assert ref.shape == (4, 128)


def test_kernel_dtype_keeps_the_input_type():
    # Outside autocast the network runs in x's own type (the reference's
    # INPUT_DTYPE kernels, mlp_fused.md:159-166): bf16, fp16 and fp32 as
    # they are, float64 in fp32 (keeping the range), other types in fp16.
    from mlpmk.autograd import kernel_dtype

    for dt, want in ((torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                     (torch.float32, torch.float32), (torch.float64, torch.float32),
                     (torch.int32, torch.float16)):
        assert kernel_dtype(torch.empty(2, 2, dtype=dt), (2, 256, 2)) == want, dt


def test_input_pad_rule():
    # Input widths that are not multiples of 16 are zero-padded to the next
    # one where the padded network has a fused forward; otherwise (too deep,
    # fp32 wider than 128, any width above 256) nothing is padded.
    from mlpmk.autograd import _input_pad

    f16, f32 = torch.float16, torch.float32
    assert _input_pad((3, 64, 64, 4), f16) == 13
    assert _input_pad((63, 128, 128, 8), torch.bfloat16) == 1
    assert _input_pad((5, 256, 256, 256, 16), f16) == 11
    assert _input_pad((3, 64, 64, 64, 16), f32) == 13
    assert _input_pad((16, 64, 64, 4), f16) == 0
    assert _input_pad((3,) + (64,) * 7 + (4,), f16) == 0
    assert _input_pad((3, 256, 256, 16), f32) == 0
    assert _input_pad((3, 320, 320, 16), f16) == 0


def test_launcher_route_rule():
    # kernel._fused_mlp_fwd's cached route per (K1, N1, N2, N3, dtype): one
    # fused launch (0), zero columns to pad x with first (> 0), or layer by
    # layer (-1); other dtypes go to the launch, which rejects them.
    f16, f32 = torch.float16, torch.float32
    assert kernel._route((128, 128, 128, 128, f16)) == 0
    assert kernel._route((3, 128, 128, 64, f16)) == 13
    assert kernel._route((3, 128, 128, 64, f32)) == 13
    assert kernel._route((3, 256, 256, 64, f32)) == -1  # fp32 wider than 128
    assert kernel._route((128, 320, 128, 128, f16)) == -1  # wider than 256
    assert kernel._route((128, 128, 128, 128, torch.int32)) == 0
