"""CPU oracle for the fused softplus-MLP hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  The product path (``mlp-megakernel_amd``) never calls into it and fails
loudly when its HIP library is missing.

It restates, in plain numpy, the math of the reference's eager path and of the
(absent-from-the-snapshot) training path described in its report:

* ``softplus``            -- ``where(z > 20, z, log(exp(z) + 1))``
                              (/root/reference/kernel.py:108,112;
                              cutile_mlp.py:38-40)
* ``forward``             -- ``h1 = softplus(x @ W1); h2 = softplus(h1 @ W2); out = h2 @ W3``
                              (kernel.py:168-171, profile.py:102-106) for any depth
                              (5-layer chain: README.md:9, mlp_fused.md:11)
* ``forward`` with ``round_hidden=True`` mirrors the megakernel's fp16 re-cast of
  every hidden activation before the next GEMM (kernel.py:110,117,121); with
  ``elem="bf16"`` the re-cast is to bf16, as the reference's ``.to(INPUT_DTYPE)``
  does for a bf16 INPUT_DTYPE (mlp_fused.md:159-163).
* ``to_bf16``             -- fp32 -> bf16 rounding (round to nearest, ties to
                              even; NaN stays NaN), values returned as fp32.
* ``backward``            -- closed form of mlp_fused.md:84-95:
                              ``dz_L = g``, ``dW_l = h_{l-1}^T dz_l``,
                              ``dz_{l-1} = (dz_l W_l^T) * (1 - exp(-h_{l-1}))``,
                              ``dx = dz_1 W_1^T``
* ``wn_forward`` / ``wn_backward`` -- weight norm ``W = g * v / ||v||`` per output
  column (mlp_fused.md:467-483, README.md:34), gradients by the chain rule.

Weights are ``[in, out]`` row-major, as kernel.py:105,109,113-114 index them.

Pinning (what checks this restatement, in tests/test_oracle.py):
  softplus  -> torch.nn.functional.softplus (library), pure-Python math.log1p/exp
               on the threshold edges, and the planted "branchless" bug of
               ablation_report.md:75-79 must fail.
  forward   -> torch CPU float64 matmul+softplus (library), closed forms
               (zero W1 gives h1 = ln 2; identity weights give softplus(softplus(x)));
               linearity in the last layer; the committed golden fixtures.
  backward  -> torch.autograd in float64 (library), central finite
               differences on tiny shapes; planted bugs must fail (dropped
               activation derivative, derivative from the wrong argument,
               W instead of W^T in the data gradient).
  wn_*      -> torch._weight_norm (library) and its autograd; invariants
               ||W[:, j]|| = |g_j|, <dv[:, j], v[:, j]> = 0.
  to_bf16   -> torch's float32 -> bfloat16 conversion (library) on random and
               edge values (ties, overflow to inf, NaN, subnormals).
No function of this module is "parity unpinned".
"""
from __future__ import annotations

import numpy as np

SOFTPLUS_THRESHOLD = 20.0  # kernel.py:108 (beta = 1, threshold = 20)
LN2 = float(np.log(2.0))


def softplus(z, dtype=np.float32):
    """``where(z > 20, z, log(exp(z) + 1))`` -- /root/reference/kernel.py:108.

    ``log1p(exp(z))`` is used for the non-linear branch, which is what
    ``torch.nn.functional.softplus`` evaluates; it differs from the literal
    ``log(exp(z) + 1)`` only below 2**-24 in absolute value.
    """
    z = np.asarray(z, dtype=dtype)
    with np.errstate(over="ignore"):
        lin = np.log1p(np.exp(np.minimum(z, SOFTPLUS_THRESHOLD)))
    return np.where(z > SOFTPLUS_THRESHOLD, z, lin).astype(dtype, copy=False)


def to_bf16(a):
    """Round fp32 values to bf16 (8 significant bits; round to nearest, ties
    to even) and return them as fp32.  Adds 0x7FFF plus the lowest kept bit
    to the bit pattern and clears the low 16 bits; NaNs are kept as NaNs."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, r).astype(np.float32)


def round_elem(a, elem):
    """``a`` rounded to the 16-bit element format ``elem`` ("f16" or "bf16"), as fp32."""
    if elem == "bf16":
        return to_bf16(a)
    if elem == "f16":
        return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    raise ValueError(f"elem must be 'f16' or 'bf16', got {elem!r}")


def softplus_grad_from_h(h, dtype=np.float32):
    """``softplus'(z) = sigmoid(z) = 1 - exp(-h)`` with ``h = softplus(z)``
    (mlp_fused.md:57,84).  Uses ``-expm1(-h)`` for accuracy at small ``h``."""
    h = np.asarray(h, dtype=dtype)
    return (-np.expm1(-h)).astype(dtype, copy=False)


def forward(x, weights, *, round_hidden=False, dtype=np.float32, return_hidden=False, elem="f16"):
    """Eager chain ``softplus(... softplus(x @ W1) ...) @ WL`` (kernel.py:168-171).

    ``x`` and ``weights`` are upcast to ``dtype`` (their fp16 values are exact in
    fp32).  With ``round_hidden`` each hidden activation is rounded to fp16
    (``elem="bf16"``: bf16) before it feeds the next GEMM, as the Triton
    megakernel's ``.to(tl.float16)`` does (kernel.py:110,117).  Returns ``out``
    (and the list of hidden activations ``[h1, ..., h_{L-1}]`` in ``dtype`` when
    ``return_hidden``).
    """
    a = np.asarray(x).astype(dtype)
    hidden = []
    nl = len(weights)
    for li, w in enumerate(weights):
        z = a @ np.asarray(w).astype(dtype)
        if li == nl - 1:
            out = z
            break
        h = softplus(z, dtype)
        hidden.append(h)
        a = round_elem(h, elem).astype(dtype) if round_hidden else h
    if return_hidden:
        return out, hidden
    return out


def backward(x, weights, hidden, dout, *, dtype=np.float32, need_dx=True):
    """Closed-form gradients of ``out = MLP(x)`` (mlp_fused.md:88-95).

    ``hidden`` are the post-activation values ``[h1, ..., h_{L-1}]`` (the fp32
    stash of README.md:30).  ``dout`` is ``dL/dout`` ``[M, OUT]``.
    Returns ``(dws, dx)`` with ``dws[l] = h_{l-1}^T @ dz_l`` (``h_0 = x``).
    """
    nl = len(weights)
    ws = [np.asarray(w).astype(dtype) for w in weights]
    acts = [np.asarray(x).astype(dtype)] + [np.asarray(h).astype(dtype) for h in hidden]
    dz = np.asarray(dout).astype(dtype)
    if dz.ndim == 1:
        dz = np.broadcast_to(dz, (acts[0].shape[0], dz.shape[0]))
    dws = [None] * nl
    for li in range(nl - 1, -1, -1):
        dws[li] = acts[li].T @ dz
        if li == 0:
            break
        dh = dz @ ws[li].T
        dz = dh * softplus_grad_from_h(acts[li], dtype)
    dx = (dz @ ws[0].T) if need_dx else None
    return dws, dx


def wn_forward(v, g, dtype=np.float32):
    """Weight norm per output column: ``W[:, j] = g_j * v[:, j] / ||v[:, j]||``
    (mlp_fused.md:467-474).  ``v`` is ``[in, out]``; returns ``(W, inv_norm)``."""
    v = np.asarray(v).astype(dtype)
    g = np.asarray(g).astype(dtype)
    norm = np.sqrt((v.astype(np.float64) ** 2).sum(axis=0)).astype(dtype)
    inv = (1.0 / norm).astype(dtype)
    return (v * (g * inv)[None, :]).astype(dtype), inv


def wn_backward(dw, v, g, dtype=np.float32):
    """Chain rule through ``W = g v / ||v||`` (mlp_fused.md:474,481-483):
    ``dg_j = <dW_j, v_j> / ||v_j||``;
    ``dv_j = (g_j / ||v_j||) (dW_j - dg_j v_j / ||v_j||)``."""
    dw = np.asarray(dw).astype(dtype)
    v = np.asarray(v).astype(dtype)
    g = np.asarray(g).astype(dtype)
    norm = np.sqrt((v.astype(np.float64) ** 2).sum(axis=0)).astype(dtype)
    inv = (1.0 / norm).astype(dtype)
    u = v * inv[None, :]
    dg = (dw * u).sum(axis=0)
    dv = (g * inv)[None, :] * (dw - dg[None, :] * u)
    return dv.astype(dtype), dg.astype(dtype)


# ---------------------------------------------------------------------------
# Seeded synthetic inputs for the BASELINE configs (shared by tests and bench)
# ---------------------------------------------------------------------------

CONFIGS = {
    # name: layer widths (D, H..., OUT) and the input distribution
    "3l128": {"dims": (128, 128, 128, 128), "x": "normal"},
    "5l128": {"dims": (128, 128, 128, 128, 128, 128), "x": "normal"},
    "narrow": {"dims": (32, 64, 64, 16), "x": "uniform"},
}


def make_inputs(dims, m, seed=0, x_dist="normal", elem="f16"):
    """fp16 ``x`` ``[m, dims[0]]`` (N(0,1) or U(-1,1)) and fp16 weights
    ``W_l ~ N(0, 1/in)`` ``[in, out]`` from one numpy generator.  With
    ``elem="bf16"`` the same draws rounded to bf16, as fp32 arrays (numpy has
    no bf16 type; the values convert exactly)."""
    rng = np.random.default_rng(seed)
    if x_dist == "normal":
        x = rng.standard_normal((m, dims[0]), dtype=np.float32)
    else:
        x = rng.uniform(-1.0, 1.0, size=(m, dims[0])).astype(np.float32)
    ws = [
        rng.standard_normal((dims[i], dims[i + 1]), dtype=np.float32) / np.sqrt(dims[i])
        for i in range(len(dims) - 1)
    ]
    if elem == "bf16":
        return to_bf16(x), [to_bf16(w) for w in ws]
    return x.astype(np.float16), [w.astype(np.float16) for w in ws]


def make_wn_params(dims, seed=0):
    """Weight-norm parameters of the training config: ``v ~ N(0, 1/in)``, ``g = 1``."""
    rng = np.random.default_rng(seed + 1000)
    vs = [
        (rng.standard_normal((dims[i], dims[i + 1]), dtype=np.float32) / np.sqrt(dims[i])).astype(np.float32)
        for i in range(len(dims) - 1)
    ]
    gs = [np.ones(dims[i + 1], dtype=np.float32) for i in range(len(dims) - 1)]
    return vs, gs


def allclose_report(got, ref, atol, rtol):
    """``(ok, max_abs_err, worst_excess)`` for ``|got-ref| <= atol + rtol*|ref|``."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    excess = float(np.max(err - bound)) if err.size else 0.0
    return bool(np.all(err <= bound)), float(err.max() if err.size else 0.0), excess
