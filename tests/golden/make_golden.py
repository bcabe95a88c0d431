"""Writes the small golden fixtures under tests/golden/.

Expected values come from torch on the CPU in float64 (F.softplus with the
reference's beta=1 / threshold=20, matmul, torch._weight_norm and autograd) --
an implementation independent of oracle/mlp_oracle.py, which the tests then
check against these files.  Inputs are the seeded fp16 tensors of the
BASELINE configs at small M.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle.mlp_oracle import make_inputs, make_wn_params  # noqa: E402  (seeded input generator only)


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def mlp(x, ws):
    a = x
    for i, w in enumerate(ws):
        a = a @ w
        if i < len(ws) - 1:
            a = F.softplus(a, beta=1.0, threshold=20.0)
    return a


def forward_fixture(name, dims, m, x_dist):
    x, ws = make_inputs(dims, m, seed=0, x_dist=x_dist)
    out = mlp(t64(x), [t64(w) for w in ws]).numpy().astype(np.float32)
    arrs = {"x": x, "out": out, "num_layers": np.int64(len(ws))}
    for i, w in enumerate(ws):
        arrs[f"w{i + 1}"] = w
    np.savez_compressed(os.path.join(HERE, name), **arrs)


def training_fixture(name, m):
    dims = (128, 128, 128, 128)
    x, _ = make_inputs(dims, m, seed=0)
    vs, gs = make_wn_params(dims)
    rng = np.random.default_rng(7)
    gs = [(g * rng.uniform(0.5, 1.5, size=g.shape)).astype(np.float32) for g in gs]
    dout = rng.standard_normal((m, dims[-1])).astype(np.float32)
    vt = [t64(v).requires_grad_(True) for v in vs]
    gt = [t64(g).requires_grad_(True) for g in gs]
    wt = [torch._weight_norm(v, g[None, :], 1) for v, g in zip(vt, gt)]
    for w in wt:
        w.retain_grad()
    xt = t64(x).requires_grad_(True)
    out = mlp(xt, wt)
    (out * t64(dout)).sum().backward()
    arrs = {"x": x, "dout": dout, "out": out.detach().numpy().astype(np.float32), "dx": xt.grad.numpy().astype(np.float32)}
    for i in range(3):
        arrs[f"v{i + 1}"] = vs[i]
        arrs[f"g{i + 1}"] = gs[i]
        arrs[f"w{i + 1}"] = wt[i].detach().numpy().astype(np.float32)
        arrs[f"dw{i + 1}"] = wt[i].grad.numpy().astype(np.float32)
        arrs[f"dv{i + 1}"] = vt[i].grad.numpy().astype(np.float32)
        arrs[f"dg{i + 1}"] = gt[i].grad.numpy().astype(np.float32)
    np.savez_compressed(os.path.join(HERE, name), **arrs)


if __name__ == "__main__":
    forward_fixture("fwd_3l128_m256.npz", (128, 128, 128, 128), 256, "normal")
    forward_fixture("fwd_5l128_m64.npz", (128,) * 6, 64, "normal")
    forward_fixture("fwd_narrow_m64.npz", (32, 64, 64, 16), 64, "uniform")
    training_fixture("train_wn_3l128_m64.npz", 64)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
