"""Drop-in for the reference's ``kernel.py`` (3-layer inference megakernel).

Same public surface as /root/reference/kernel.py:
  * ``_fused_mlp_fwd(x, w1, w2, w3) -> out``  (kernel.py:130-156): contiguous
    copies of the inputs, a fresh ``[M, N3]`` output of x's dtype (fp16, bf16
    or fp32, as the reference passes fp32 on, kernel.py:138), one
    asynchronous launch on the current stream, no synchronisation.
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
# fwd_dispatch / launch_fwd_any and fwd_split.hip fwd_split_dispatch).  On a
# GPU, _pick_config asks the library (mlpmk_fwd_launch_info, the same code
# path that launches); this mirror answers without a device.
_MI355X_CUS = 256
# dims -> (max 32-row blocks per CU for the feature-split kernel, its waves,
#          rows per block of the persistent kernel, its largest waves per workgroup)
_POLICY = {
    (128, 128, 128, 128): (1, 4, 32, 12),
    (128, 128, 128, 128, 128, 128): (2, 4, 32, 12),
    (32, 64, 64, 16): (2, 2, 64, 16),
}
_GENERIC_POLICY = (0, 0, 32, 8)  # runtime-width kernels: no split kernel, at most 8 waves
# fp32 tensors (fwd_x3.hip): the feature-split kernels at every M, 32-row
# blocks; 4 waves per layer (one per 32 output features of a 128-wide layer;
# the runtime-width kernels are compiled at width 128), one wave group per
# layer for 2 and 3 layers (the layer pipeline), one group running every
# layer for 4 and 5.
_F32_WAVES_PER_LAYER = 4


def _f32_waves(n_layers):
    return _F32_WAVES_PER_LAYER * (n_layers if n_layers <= 3 else 1)


def __getattr__(name):
    if name == "NUM_SMS":
        return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    raise AttributeError(name)


def _mirror_policy(M, dims, num_cus, fp32=False):
    if max(dims) > 128:  # streamed-weight kernel (fwd_wide.hip): 32-row blocks, 8 waves from 256 rounds
        return 32, (4 if M < 256 * num_cus else 8)
    if fp32:
        return 32, _f32_waves(len(dims) - 1)
    split_per_cu, split_waves, bm, max_waves = _POLICY.get(tuple(dims), _GENERIC_POLICY)
    if -(-M // 32) <= split_per_cu * num_cus:
        return 32, split_waves
    blocks = -(-M // bm)
    if max_waves > 4 and blocks <= 4 * num_cus:
        return bm, 4
    if max_waves > 8 and blocks <= 8 * num_cus:
        return bm, 8
    return bm, max_waves


def _pick_config(M, K1, N1, N2, N3, fp32=False, num_cus=None):
    """gfx950 launch policy in the reference's tuple shape
    ``(BM, BN3, BK1, BK2, BK3, warps)`` (kernel.py:25-53) for the 3-layer
    network ``K1 -> N1 -> N2 -> N3`` at batch M.

    BM = rows per MFMA batch block (32; 64 for the narrow network's
    persistent kernel, which reads each weight fragment for two blocks),
    BN3 = the whole output width (a workgroup computes every output column),
    BK* = 16 (the K of v_mfma_f32_32x32x16_f16), warps = 64-lane waves per
    workgroup:
      * small batches (up to one 32-row block per CU for 3L-128, two for the
        narrow network): the feature-split kernel, one wave per 32 output
        features (4 waves; 2 for the narrow network) sharing each block;
      * otherwise the persistent kernel with 4 waves per workgroup up to 4
        blocks per CU, 8 up to 8, then 12 (16 narrow); runtime-width
        networks (any other widths) at most 8.
    Widths above 128 (up to 256) take the streamed-weight kernel at every M
    (8 waves, one 32-row block each per round).
    With ``num_cus`` None and a GPU present the answer comes from the library
    (``mlpmk_fwd_launch_info``); otherwise from the mirror above with
    ``num_cus`` CUs (MI355X's 256 by default).  ``fp32`` inputs (fp32 x, W
    and out; bf16 hi/lo split MFMA operands) always take their feature-split
    kernel: 32-row blocks, 4 waves.  fp32 networks wider than 128 have no
    fused kernel (``_fused_mlp_fwd`` runs them layer by layer): the library
    query raises ``MlpmkError`` for them.
    """
    dims = (K1, N1, N2, N3)
    if num_cus is None and torch.cuda.is_available():
        info = _ops.fwd_launch_info(dims, max(int(M), 1), dtype=torch.float32 if fp32 else torch.float16)
        return info["rows_per_block"], N3, 16, 16, 16, info["waves"]
    bm, warps = _mirror_policy(M, dims, _MI355X_CUS if num_cus is None else num_cus, fp32=fp32)
    return bm, N3, 16, 16, 16, warps


# (K1, N1, N2, N3, dtype) -> how _fused_mlp_fwd runs it: 0 one fused launch
# (also every other dtype, which fwd_into rejects with its own message), a
# positive count of zero columns to pad x with first, -1 layer by layer.  The
# library's answer is cached: asking it costs ~2 us of ctypes per call.
_ROUTES = {}


def _route(key):
    *dims, dt = key
    if dt not in (torch.float32, torch.float16, torch.bfloat16) or _ops.fwd_supported(dims, dt):
        return 0
    pad = -dims[0] % 16
    if pad and _ops.fwd_supported([dims[0] + pad] + dims[1:], dt):
        return pad
    return -1


def _fused_mlp_fwd(x, w1, w2, w3):
    """Inference forward: one kernel launch, no intermediate in global memory
    (an input width that is not a multiple of 16 is zero-padded to one first;
    networks no fused kernel takes -- fp32 ones wider than 128, any wider
    than 256 -- run layer by layer: mlpmk.fallback.fwd)."""
    x = x.contiguous()
    w1, w2, w3 = w1.contiguous(), w2.contiguous(), w3.contiguous()
    M = x.shape[0]
    N3 = w3.shape[1]
    key = (x.shape[1], w1.shape[1], w2.shape[1], N3, x.dtype)
    route = _ROUTES.get(key)
    if route is None:
        route = _ROUTES[key] = _route(key)
    if route > 0:
        # Input width not a multiple of 16: zero columns of x and zero rows of
        # W1 add nothing to x @ W1.
        x, w1 = F.pad(x, (0, route)), F.pad(w1, (0, 0, 0, route))
    elif route < 0:
        from mlpmk import fallback

        return fallback.fwd(x, [w1, w2, w3])
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
