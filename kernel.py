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

The launch goes to the hand-written gfx950 HIP megakernels in ``libmlpmk.so``
(``mlp-megakernel_amd/csrc/fwd.hip``, ``fwd_split.hip`` for small batches)
through its C ABI.  There is no Triton
and no fallback: without the library every call raises.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

import _mlpmk  # noqa: F401  (registers the package as ``mlpmk``)
from mlpmk import ops as _ops

# gfx950 launch policy of the inference forward (mlp-megakernel_amd/csrc/fwd.hip
# and fwd_split.hip), mirrored here for _pick_config.
_MI355X_CUS = 256
_WAVES_PER_WG_WIDE = 12  # one-block-per-wave kernel, 3 waves per SIMD
_WAVES_PER_WG_NARROW = 16


def __getattr__(name):
    if name == "NUM_SMS":
        return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    raise AttributeError(name)


def _pick_config(M, K1, N1, N2, N3, fp32=False, num_cus=None):
    """gfx950 launch policy in the reference's tuple shape
    ``(BM, BN3, BK1, BK2, BK3, warps)`` (kernel.py:25-53), as the library
    applies it for the 3-layer network at this M.

    BM = rows per block (32: one MFMA batch block; 64 for the narrow network's
    one-block-per-wave kernel, which reads each weight fragment for two
    blocks), BN3 = the whole output width (a workgroup computes every output
    column), BK* = 16 (the K of v_mfma_f32_32x32x16_f16), warps = 64-lane waves
    per workgroup:
      * up to one 32-row block per CU (two for the narrow network): the
        feature-split kernel, one wave per 32 output features (4 waves, 2 for
        the narrow network) sharing each block;
      * otherwise the persistent one-block-per-wave kernel with 4 waves per
        workgroup up to 4 blocks per CU, 8 up to 8, then 12 (16 narrow).
    ``num_cus`` defaults to ``NUM_SMS`` on a GPU and to MI355X's 256
    otherwise.  ``fp32`` inputs are not supported by the main-branch surface
    either (/root/reference/AGENTS.md:86-88).
    """
    if fp32:
        raise TypeError("the fused forward takes fp16 inputs (main-branch surface is fp16 only)")
    if num_cus is None:
        num_cus = NUM_SMS if torch.cuda.is_available() else _MI355X_CUS  # noqa: F821 (module __getattr__)
    narrow = max(K1, N1, N2, N3) <= 64
    if -(-M // 32) <= (2 if narrow else 1) * num_cus:
        return 32, N3, 16, 16, 16, 2 if narrow else 4
    bm = 64 if narrow else 32
    blocks = -(-M // bm)
    warps = 4 if blocks <= 4 * num_cus else 8 if blocks <= 8 * num_cus else (
        _WAVES_PER_WG_NARROW if narrow else _WAVES_PER_WG_WIDE)
    return bm, N3, 16, 16, 16, warps


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
