"""Drop-in for the reference's ``fused_mlp.py`` training modules
(/root/reference/README.md:18,58-70; the file itself is not in the reference
snapshot, so the constructor signature follows the README quick start and the
parameter layout follows /root/reference/mlp_fused.md:478-480).

    from fused_mlp import FusedMLPSoftplus, FusedMLPSoftplusWN
    model = FusedMLPSoftplus(D=128, H=128, out_features=128).cuda().half()
    out = model(x)            # one forward-megakernel launch
    out.sum().backward()      # one backward-megakernel launch

Network: ``out = softplus(softplus(x @ W1) @ W2) @ W3``, no bias, softplus with
beta = 1 and threshold = 20.  Weights are stored ``[in, out]`` (the layout the
megakernel indexes, /root/reference/kernel.py:105,109,113-114).  The
gfx950 kernels behind the modules live in ``mlp-megakernel_amd/csrc``; the
modules raise if the library is missing (there is no eager fallback).

Initialisation (not stated by the reference): ``W ~ N(0, 1/in)``; with weight
norm ``v ~ N(0, 1/in)`` and ``g = 1`` (the training configuration of this
build's benchmark).
"""
import math

import torch
import torch.nn as nn

import _mlpmk  # noqa: F401  (registers the package as ``mlpmk``)
from mlpmk.autograd import FusedMLPFunction, FusedMLPWNFunction, _split, fused_mlp, fused_mlp_wn  # noqa: F401


def _dims(D, H, out_features, n_layers):
    return (D,) + (H,) * (n_layers - 1) + (out_features,)


class FusedMLPSoftplus(nn.Module):
    """Softplus MLP with ``n_layers`` bias-free layers (3 by default), fused
    forward and backward on MI355X."""

    def __init__(self, D=128, H=128, out_features=128, n_layers=3):
        super().__init__()
        self.dims = _dims(D, H, out_features, n_layers)
        self.weights = nn.ParameterList(
            [nn.Parameter(torch.randn(self.dims[i], self.dims[i + 1]) / math.sqrt(self.dims[i]))
             for i in range(n_layers)]
        )

    def forward(self, x):
        # The network runs in mlpmk.autograd.kernel_dtype(x): the autocast
        # dtype under autocast, else x's own type (bf16, fp16 or fp32; fp32
        # through bf16 hi/lo split operands) and fp16 for anything else;
        # networks no fused kernel takes (fp32 wider than 128, any wider
        # than 256) run layer by layer in that type; autograd carries the
        # gradient back through the casts.  Without autograd (no_grad, inference_mode, or
        # nothing requiring grad) this is one plain forward launch, no stash.
        return fused_mlp(x, *self.weights)

    def extra_repr(self):
        return f"dims={self.dims}"


class FusedMLPSoftplusWN(nn.Module):
    """Weight-normalised variant: ``W_l[:, j] = g_l[j] v_l[:, j] / ||v_l[:, j]||``
    per output column, all layers' ``v`` in one contiguous block ``v_all`` and all
    ``g`` in ``g_all``.  Forward: one weight-norm launch + one megakernel launch;
    backward: one megakernel launch + one weight-norm launch."""

    def __init__(self, D=128, H=128, out_features=128, n_layers=3):
        super().__init__()
        self.dims = _dims(D, H, out_features, n_layers)
        d = self.dims
        self.v_all = nn.Parameter(
            torch.cat([(torch.randn(d[i], d[i + 1]) / math.sqrt(d[i])).reshape(-1) for i in range(n_layers)])
        )
        self.g_all = nn.Parameter(torch.ones(sum(d[1:])))

    def v(self, layer):
        """View of layer ``layer``'s direction matrix ``[in, out]``."""
        return _split(self.v_all, self.dims)[layer]

    def g(self, layer):
        """View of layer ``layer``'s magnitudes ``[out]``."""
        off = sum(self.dims[1 : 1 + layer])
        return self.g_all[off : off + self.dims[layer + 1]]

    def forward(self, x):
        # Element type and stash rule as FusedMLPSoftplus.forward.
        return fused_mlp_wn(x, self.v_all, self.g_all, self.dims)

    def extra_repr(self):
        return f"dims={self.dims}"
