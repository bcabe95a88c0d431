"""Drop-in for the reference's ``kernel.py`` (3-layer inference megakernel).

Same public surface as /root/reference/kernel.py:
  * ``_fused_mlp_fwd(x, w1, w2, w3) -> out``  (kernel.py:130-156): contiguous
    copies of the inputs, a fresh fp16 ``[M, N3]`` output, one asynchronous
    launch on the current stream, no synchronisation.
  * ``_pick_config(M, K1, N1, N2, N3, fp32=False)`` (kernel.py:25-53): the
    launch policy, here the gfx950 one.
  * ``Model`` (eager reference, kernel.py:163-171) and ``ModelNew`` (fused,
    kernel.py:174-180).
  * ``NUM_SMS`` (kernel.py:18) is read lazily on first access instead of at
    import, so importing this module needs no GPU.

The launch goes to the hand-written gfx950 HIP megakernel in ``libmlpmk.so``
(``mlp-megakernel_amd/csrc/fwd.hip``) through its C ABI.  There is no Triton
and no fallback: without the library every call raises.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

import _mlpmk  # noqa: F401  (registers the package as ``mlpmk``)
from mlpmk import ops as _ops

# Waves per workgroup of the gfx950 inference forward (mlp-megakernel_amd/csrc/fwd.hip):
# 12 (3 per SIMD) for 128-wide layers, 16 for the narrow network.
_WAVES_PER_WG_WIDE = 12
_WAVES_PER_WG_NARROW = 16


def __getattr__(name):
    if name == "NUM_SMS":
        return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    raise AttributeError(name)


def _pick_config(M, K1, N1, N2, N3, fp32=False):
    """gfx950 launch policy in the reference's tuple shape
    ``(BM, BN3, BK1, BK2, BK3, warps)`` (kernel.py:25-53).

    BM = rows a wave computes per block (32: one MFMA batch block), BN3 = the whole
    output width (one pass computes every output column), BK* = 16 (the K of
    v_mfma_f32_32x32x16_f16), warps = 64-lane waves per workgroup.  The
    persistent grid is min(CUs x occupancy, ceil(M / (BM * warps))) and the
    waves of a workgroup claim its row blocks from an LDS counter.  ``fp32``
    inputs are not supported by the main-branch surface either
    (/root/reference/AGENTS.md:86-88).
    """
    if fp32:
        raise TypeError("the fused forward takes fp16 inputs (main-branch surface is fp16 only)")
    narrow = max(K1, N1, N2, N3) <= 64
    return 32, N3, 16, 16, 16, _WAVES_PER_WG_NARROW if narrow else _WAVES_PER_WG_WIDE


def _fused_mlp_fwd(x, w1, w2, w3):
    """Inference forward: one kernel launch, no intermediate in global memory."""
    x = x.contiguous()
    w1, w2, w3 = w1.contiguous(), w2.contiguous(), w3.contiguous()
    M = x.shape[0]
    N3 = w3.shape[1]
    out = torch.empty((M, N3), device=x.device, dtype=x.dtype)
    _ops.fwd_into(x, [w1, w2, w3], out)
    return out


class Model(nn.Module):
    """PyTorch reference: 3-layer MLP with softplus."""

    def __init__(self):
        super().__init__()

    def forward(self, x, w1, w2, w3):
        h1 = F.softplus(x @ w1)
        h2 = F.softplus(h1 @ w2)
        return h2 @ w3


class ModelNew(nn.Module):
    """Fused gfx950 megakernel: 3-layer MLP with softplus."""

    def __init__(self):
        super().__init__()

    def forward(self, x, w1, w2, w3):
        return _fused_mlp_fwd(x, w1, w2, w3)
