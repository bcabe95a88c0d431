"""Drop-in for the reference's ``fused_mlp5.py`` (5-layer variant,
/root/reference/README.md:9,19; /root/reference/mlp_fused.md:38,75-76 -- the
file is not in the snapshot and its class names are not documented, so the
names here are this build's).

    out = softplus(softplus(softplus(softplus(x@W1)@W2)@W3)@W4)@W5

The 5-layer forward runs on the gfx950 forward megakernel (all five 128x128
weight matrices staged in the 160 KiB LDS).  The backward is two launches of
the backward megakernel -- layers 4..2, whose fp16 gradient of h_1 goes
through a workspace to layers 1..0 -- since four dgrad weight blocks and the
exchange tiles do not fit one workgroup's LDS together.
"""
import _mlpmk  # noqa: F401
from fused_mlp import FusedMLPSoftplus, FusedMLPSoftplusWN


class FusedMLP5Softplus(FusedMLPSoftplus):
    """Five bias-free softplus layers, fused forward and backward."""

    def __init__(self, D=128, H=128, out_features=128):
        super().__init__(D, H, out_features, n_layers=5)


class FusedMLP5SoftplusWN(FusedMLPSoftplusWN):
    """Weight-normalised five-layer variant."""

    def __init__(self, D=128, H=128, out_features=128):
        super().__init__(D, H, out_features, n_layers=5)
