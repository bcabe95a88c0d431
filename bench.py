"""Benchmark of the gfx950 fused softplus-MLP megakernels.

Headline (throughput point): the 3-layer
D=H=OUT=128 fp16 forward at M = 1,048,576 rows, seeded synthetic inputs
(x ~ N(0,1), W_l ~ N(0, 1/in)) resident in HBM before timing.  A "step" is one
launch over the whole batch.  Two input/output buffer pairs alternate so the
1 GiB working set cannot sit in the 256 MB Infinity Cache.  ``value`` and
``roofline`` come from the K timed launches (HIP events around them, after a
0.1 s clock ramp and W warm-up launches); ``sustained`` repeats the
measurement over >= 0.5 s of back-to-back launches.

Besides the headline the default run times every other BASELINE config (extra
keys, each with the buffers it touches rotated past the Infinity Cache or
labelled cache-resident): the 5-layer and narrow forwards, M = 65,536, the
M = 64..4096 latency sweep (event timing, one-launch and 20-launch graph
replays, and the replay floor of a one-workgroup kernel), and the
weight-norm training step at M = 4096 / 16384 / 131072.  ``cpu_baseline`` is
the reference's eager PyTorch path (kernel.py:163-171) in fp32 on the host
cores over the workload itself (all M rows of the seed-0 inputs the GPU
reads; median of at least 3 passes); the numpy oracle's time is reported
beside it.

Prints ONE JSON line (the driver's contract).  ``--config`` / ``--m`` move the
headline to another config, ``--no-extra`` skips the extra configs (for
profiler runs), ``--train`` adds the longer training experiments.
"""
import argparse
import contextlib
import gc
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fwd rows/s + % of fp16 MFMA/HBM roofline, 3-layer 128-wide MLP, M=64..1M"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
MFMA_F16_PEAK_TFLOPS = 2516.6  # MI355X dense fp16, published (2.5 PF)

CONFIG_DIMS = {
    "3l128": (128, 128, 128, 128),
    "5l128": (128, 128, 128, 128, 128, 128),
    "narrow": (32, 64, 64, 16),
    # hidden width 256 (streamed-weight kernel; not a BASELINE config)
    "3l256": (128, 256, 256, 128),
}
DEFAULT_M = {"3l128": 1048576, "5l128": 1048576, "narrow": 4194304, "3l256": 1048576}


def algorithmic(dims, m, esize=2):
    """(bytes, flops) of one forward launch: x + out rows once, weights once
    (``esize`` bytes per element: 2 for fp16/bf16 tensors, 4 for fp32)."""
    wbytes = esize * sum(dims[i] * dims[i + 1] for i in range(len(dims) - 1))
    rbytes = esize * (dims[0] + dims[-1])
    flops = 2 * sum(dims[i] * dims[i + 1] for i in range(len(dims) - 1))
    return rbytes * m + wbytes, flops * m


def make_device_inputs(torch, dims, m, seed, uniform):
    g = torch.Generator(device="cuda").manual_seed(seed)
    if uniform:
        x = (torch.rand((m, dims[0]), generator=g, device="cuda") * 2 - 1).half()
    else:
        x = torch.randn((m, dims[0]), generator=g, device="cuda").half()
    ws = [
        (torch.randn((dims[i], dims[i + 1]), generator=g, device="cuda") / dims[i] ** 0.5).half()
        for i in range(len(dims) - 1)
    ]
    return x, ws


@contextlib.contextmanager
def gc_paused():
    """Python's garbage collector off for the block (as timeit does), after
    one collection up front: a generation-2 collection with torch loaded
    stalls the launching thread for 25-40 ms, long enough for the GPU to
    drain its queue in the middle of a timed region, and a collection between
    the clock ramp and the timed launches idles the GPU long enough for its
    clock to drop again."""
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


def ramp_clock(torch, fn, seconds=0.1):
    """Untimed back-to-back launches for about `seconds`, enqueued without
    host synchronisation, so that the timed launches do not start from the
    idle shader clock (~150 launches of the 3-layer forward to settle).  Kept
    short: under seconds of continuous load the MI355X power management
    lowers the clock (measured: the 3-layer forward drifts from ~127 to
    ~140 us per launch over 0.5 s)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(10):
        fn(i)
    torch.cuda.synchronize()
    per_launch = max((time.perf_counter() - t0) / 10, 1e-6)
    for i in range(min(int(seconds / per_launch), 20000)):
        fn(i)
    torch.cuda.synchronize()


def time_launches(torch, fn, steps, warmup):
    """Average ms per launch over `steps` back-to-back launches, bracketed by
    HIP events on the launch stream (torch's current stream).  Callers run it
    inside gc_paused()."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_graph(torch, fn, iters=100, warmup=20, per_graph=1):
    """Median ms per launch over graph replays of `per_graph` back-to-back
    launches.  per_graph = 1 is what /root/reference/profile.py:50-80 measures
    (one launch per replay); on ROCm a replay itself costs ~15-20 us of launch
    latency, so per_graph = 20 is reported beside it as the kernel's
    launch-overhead-free time."""
    for i in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(per_graph):
            fn(i)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    for _ in range(iters):
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / per_graph)
    ts.sort()
    return ts[len(ts) // 2]


def time_per_call(torch, fn, warmup=50, iters=100):
    """Median ms of one call: an event pair recorded around each call, then a
    synchronisation, after `warmup` calls -- the reference's
    ``benchmark_fn`` (/root/reference/profile.py:28-47), which its "non-graph
    incl. launch" tables use.  Host dispatch and the allocation of the
    output are inside the pair."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    ts = []
    for _ in range(iters):
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b))
    ts.sort()
    return ts[len(ts) // 2]


def cpu_threads():
    try:
        from threadpoolctl import threadpool_info

        return max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        return os.cpu_count() or 1


def cpu_model_name():
    """The host CPU's model name (/proc/cpuinfo), as lscpu reports it."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def host_threads():
    """Host threads for the CPU legs: the CPUs this process may run on, capped
    by OMP_NUM_THREADS when set (the GPU box sets it to its CPU share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(n, 1)


def _median_runs(fn, runs, budget_s):
    """Wall-clock seconds of `runs` calls of `fn` (after one untimed call),
    stopping early once `budget_s` has elapsed with at least 3 runs done;
    returns (median, list of run times)."""
    fn()
    ts = []
    t_all = time.perf_counter()
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if len(ts) >= 3 and time.perf_counter() - t_all >= budget_s:
            break
    srt = sorted(ts)
    return srt[len(srt) // 2], ts


def cpu_oracle_numpy(orc, x, ws, runs=3, budget_s=10.0):
    """The numpy oracle's forward (fp32, BLAS matmuls) on the host over the
    workload's own inputs (the same seeded fp16 values the GPU reads):
    median of `runs` full passes."""
    threads = cpu_threads()
    med, ts = _median_runs(lambda: orc.forward(x, ws), runs, budget_s)
    m = x.shape[0]
    return {
        "value": m / med,
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "sample": f"numpy oracle fp32 forward over all {m} rows of the workload's seed-0 inputs, median of "
        f"{len(ts)} runs ({', '.join(f'{t:.3f}' for t in ts)} s; BLAS matmuls threaded, softplus "
        f"single-threaded numpy)",
    }


def cpu_eager_baseline(torch, x_dev, ws_dev, runs=5, budget_s=20.0):
    """The reference's eager path on the host: ``Model.forward``
    (kernel.py:163-171, softplus(x @ w1) -> softplus(. @ w2) -> . @ w3) in
    PyTorch fp32 on the CPU, over the workload itself -- all M rows of the
    same seed-0 inputs the GPU launch reads, upcast to fp32 -- as the median
    of `runs` full passes (at least 3)."""
    import kernel

    threads = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        x = x_dev.float().cpu()
        ws = [w.float().cpu() for w in ws_dev]
        F = torch.nn.functional
        model = kernel.Model()

        def run():
            if len(ws) == 3:
                return model(x, *ws)
            a = x  # the same chain for other depths
            for i, w in enumerate(ws):
                a = a @ w
                if i < len(ws) - 1:
                    a = F.softplus(a)
            return a

        with torch.no_grad():
            med, ts = _median_runs(run, runs, budget_s)
    finally:
        torch.set_num_threads(prev)
    m = x.shape[0]
    return {
        "value": m / med,
        "unit": "rows/s",
        "cores": threads,
        "kind": "reference",
        "cpu": cpu_model_name(),
        "sample": f"the reference's eager Model.forward (kernel.py:163-171) in PyTorch fp32 on {threads} host "
        f"threads over all {m} rows of the workload's seed-0 inputs (upcast from fp16), median of {len(ts)} "
        f"runs ({', '.join(f'{t:.3f}' for t in ts)} s)",
    }


def fwd_bench(torch, ops, dims, m, uniform, steps=200, warmup=20, dtype=None):
    """Forward launches of one config, buffers rotated so that the inputs and
    outputs they touch exceed the 256 MB Infinity Cache (>= 512 MB in
    total, at least two pairs): ms per launch (HIP events around `steps`
    launches after a 0.1 s clock ramp), rows/s, roofline fraction."""
    dtype = dtype or torch.float16
    esize = torch.empty((), dtype=dtype).element_size()
    per_pair = m * (dims[0] + dims[-1]) * esize
    pairs = max(2, -(-(512 << 20) // per_pair))
    xs, ws = [], None
    for k in range(pairs):
        x, w = make_device_inputs(torch, dims, m, seed=k, uniform=uniform)
        xs.append(x.to(dtype))
        ws = ws or [t.to(dtype) for t in w]
    outs = [torch.empty((m, dims[-1]), device="cuda", dtype=dtype) for _ in range(pairs)]

    def step(i):
        ops.fwd_into(xs[i % pairs], ws, outs[i % pairs])

    with gc_paused():
        ramp_clock(torch, step)
        ms = time_launches(torch, step, steps, warmup)
    nbytes, nflops = algorithmic(dims, m, esize)
    ai = nflops / nbytes
    hbm_bound = HBM_PEAK_GBS * ai / 1e3 < MFMA_F16_PEAK_TFLOPS
    gbs = nbytes / (ms * 1e-3) / 1e9
    tflops = nflops / (ms * 1e-3) / 1e12
    info = ops.fwd_launch_info(dims, m, dtype=dtype)
    del xs, outs
    return {
        "dtype": str(dtype).replace("torch.", ""),
        "ms_per_step": round(ms, 5),
        "rows_per_s": round(m / (ms * 1e-3), 1),
        "achieved_gbs": round(gbs, 1),
        "tflops": round(tflops, 1),
        "bound": "hbm" if hbm_bound else "mfma",
        "roofline_frac": round(gbs / HBM_PEAK_GBS if hbm_bound else tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "buffers": f"{pairs} rotating x/out pairs, {pairs * per_pair / 2**20:.0f} MiB",
        "launch": info,
    }


def latency_sweep(torch, ops, dims, sizes=(64, 128, 256, 512, 1024, 2048, 4096)):
    """BASELINE configs[1]'s latency sweep: per M, HIP-event time of 200
    back-to-back launches (host dispatch included), the median of one-launch
    graph replays (/root/reference/profile.py:50-80), 20-launch graph replays
    (launch latency shared), and the median per-call time of
    ``kernel._fused_mlp_fwd`` (``.contiguous()``, output allocation and
    launch inside an event pair, synchronised per call:
    /root/reference/profile.py:28-47); plus the replay floor of a
    one-workgroup kernel (a 16-byte copy) under the two replay methods.  Buffers are
    L2/MALL-resident at these sizes (at most 2 MiB): the figures are
    launch-latency-bound, not bandwidth measurements."""
    import kernel

    res = {}
    for m in sizes:
        x, ws = make_device_inputs(torch, dims, m, seed=0, uniform=False)
        o = torch.empty((m, dims[-1]), device="cuda", dtype=torch.float16)
        fn = lambda i: ops.fwd_into(x, ws, o)  # noqa: E731
        with gc_paused():
            ev = time_launches(torch, fn, 200, 20)
            g1 = time_graph(torch, fn)
            g20 = time_graph(torch, fn, iters=50, per_graph=20)
            call = None
            if len(ws) == 3:  # the drop-in launcher as a reference user calls it
                call = time_per_call(torch, lambda: kernel._fused_mlp_fwd(x, *ws))
        res[str(m)] = {"event_ms": round(ev, 5), "graph1_ms": round(g1, 5), "graph20_ms_per_launch": round(g20, 5),
                       "per_call_ms": None if call is None else round(call, 5),
                       "rows_per_s": round(m / (min(ev, g1, g20) * 1e-3), 1),
                       "kernel": ops.fwd_launch_info(dims, m)["kernel"]}
    src = torch.zeros(16, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    fn = lambda i: ops.copy_bytes(src, dst)  # noqa: E731
    with gc_paused():
        res["floor_one_workgroup_kernel"] = {"graph1_ms": round(time_graph(torch, fn), 5),
                                             "graph20_ms_per_launch": round(time_graph(torch, fn, iters=50, per_graph=20), 5)}
    res["note"] = "cache-resident (<= 2 MiB per M): launch-latency-bound sizes"
    return res


def sustained(torch, step, ms_hint, seconds=0.6):
    """ms per launch over >= `seconds` of back-to-back launches (one HIP-event
    pair around all of them), right after the burst measurement."""
    n = max(int(seconds / (ms_hint * 1e-3)), 100)
    with gc_paused():
        ms = time_launches(torch, step, n, 0)
    return ms, n


def train_step_bench(torch, m, steps=50, warmup=10, n_layers=3, recompute=None, dtype=None, hidden=128):
    """One training step of BASELINE config 5 through the drop-in module:
    weight norm + forward megakernel (fp32 stash), loss = out.sum(), backward
    megakernel + weight-norm backward, x without grad.  Timed with HIP events
    around `steps` back-to-back autograd steps (Python dispatch included), and
    around `steps` replays of the whole step captured as one HIP graph.
    ``dtype`` is x's type (fp32 x with the module's fp32 parameters runs the
    fp32-tensor kernels); ``hidden`` the hidden width H."""
    import fused_mlp
    from mlpmk import autograd as mag

    policy = mag.RECOMPUTE
    if recompute is not None:
        mag.RECOMPUTE = recompute
    try:
        return _train_step_bench(torch, fused_mlp, m, steps, warmup, n_layers, dtype or torch.float16, hidden)
    finally:
        mag.RECOMPUTE = policy


def _train_step_bench(torch, fused_mlp, m, steps, warmup, n_layers, dtype, hidden=128):
    from mlpmk import autograd as mag

    torch.manual_seed(0)
    model = fused_mlp.FusedMLPSoftplusWN(H=hidden, n_layers=n_layers).cuda()
    dims = tuple(model.dims)
    kdt = mag.kernel_dtype(torch.empty(0, dtype=dtype), dims)
    rc = mag._use_recompute(dims, m, False, kdt)
    # Steps rotate over nx inputs (up to 256 MB of x, at most 8 buffers) so
    # that x is not re-read from the Infinity Cache; the stash a step's
    # forward writes is read back by the same step's backward, as in training.
    nx = min(8, max(1, -(-(256 << 20) // (m * 256))))
    xs = [torch.randn(m, 128, device="cuda").to(dtype) for _ in range(nx)]  # bf16 x runs the bf16 kernels

    def step(i):
        model.v_all.grad = None
        model.g_all.grad = None
        model(xs[i % nx]).sum().backward()

    with gc_paused():
        ramp_clock(torch, step, seconds=0.2)
        ms = time_launches(torch, step, steps, warmup)

    # The same step captured whole into one HIP graph per input (the library
    # allocates nothing and records no memset); a replay costs launch latency
    # plus the kernels, no Python or autograd dispatch.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    # The graphs share one memory pool, so their intermediates (stash, dz,
    # output) reuse the same blocks as the eager steps do; they are replayed
    # in capture order, which is what sharing a pool requires.
    graphs = []
    for k in range(nx):
        model.v_all.grad = None
        model.g_all.grad = None
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=graphs[0].pool() if graphs else None):
            model(xs[k]).sum().backward()
        graphs.append(g)
    def replay(i):
        graphs[i % nx].replay()

    with gc_paused():  # the captures idled the GPU: ramp its clock again first
        ramp_clock(torch, replay, seconds=0.2)
        gms = time_launches(torch, replay, steps, warmup)
    # per row: x + out + stash written in the forward; dout, stash, x read
    # back (no dx).  Flops: forward 2*sum(in*out), dgrad of layers 1.., wgrad
    # (+ the recomputed layer).
    es = torch.empty((), dtype=kdt).element_size()
    stash_w = sum(dims[1:-1]) - (dims[-2] if rc else 0)
    nbytes = es * dims[0] + es * dims[-1] + 4 * stash_w + es * dims[-1] + 4 * stash_w + es * dims[0]
    lflop = [2 * dims[i] * dims[i + 1] for i in range(n_layers)]
    flop = sum(lflop) + sum(lflop[1:]) + sum(lflop) + (lflop[-2] if rc else 0)  # fwd, dgrad (no dx), wgrad
    return {
        "ms_per_step": round(ms, 5),
        "rows_per_s": m / (ms * 1e-3),
        "achieved_gbs": round(nbytes * m / (ms * 1e-3) / 1e9, 1),
        "tflops": round(flop * m / (ms * 1e-3) / 1e12, 2),
        "graph_ms_per_step": round(gms, 5),
        "graph_rows_per_s": m / (gms * 1e-3),
        "graph_roofline_frac": round(nbytes * m / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "launches": "wn_fwd + fwd(stash) + bwd (writes dW) + wn_bwd" if n_layers == 3 else
                    "wn_fwd + fwd(stash) + bwd (layers 4..3 write dW, then 2..0) + wn_bwd",
        "x_buffers": nx,
        "recompute_h_last": rc,
        "dims": list(dims),
        "dtype": str(kdt).replace("torch.", ""),
    }


def backward_comparison(torch, ops, m, steps=50, warmup=10):
    """The 3-layer backward at M rows, loss = out.sum(): the library's fused
    backward (mlpmk_bwd_ws + combine, writing dW, as the autograd Functions do)
    beside the reference's large-M fallback restated with PyTorch GPU ops
    (/root/reference/mlp_fused.md:114-146: data-gradient GEMMs on
    rocBLAS/hipBLASLt in fp16 with fp32 accumulation, weight-gradient GEMMs
    in fp32, the sigmoid-times-gradient step as one elementwise expression,
    weight gradients interleaved with the data gradients).  Both
    read the same fp32 stash written by the library's training forward; HIP
    events around `steps` back-to-back calls, eager and as a replayed graph."""
    dims = (128, 128, 128, 128)
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((m, 128), generator=g, device="cuda").half()
    ws = [(torch.randn((128, 128), generator=g, device="cuda") / 128 ** 0.5).half() for _ in range(3)]
    _, hs = ops.fwd(x, ws, stash=True)
    dout = torch.ones((1, 128), dtype=torch.float16, device="cuda").expand(m, 128)
    dws = [torch.zeros((128, 128), dtype=torch.float32, device="cuda") for _ in range(3)]

    def library(_):
        ops.bwd(x, ws, hs, dout, dws, accumulate=False)

    h1, h2 = hs
    wts = [w.t().contiguous() for w in ws]  # W^T, as the fallback keeps them for dgrad
    out_t = {}

    def fallback(_):
        # data gradients as fp16 GEMMs; weight gradients in fp32 (sums over
        # M rows overflow fp16 beyond ~1e4 rows), from the fp32 stash
        grad = dout.contiguous()
        dh2 = grad @ wts[2]
        out_t["dw3"] = h2.t() @ grad.float()
        dz2 = (1 - torch.exp(-h2)) * dh2
        dh1 = dz2.half() @ wts[1]
        out_t["dw2"] = h1.t() @ dz2
        dz1 = (1 - torch.exp(-h1)) * dh1
        out_t["dw1"] = x.float().t() @ dz1

    res = {}
    for name, fn in (("library", library), ("pytorch_fallback", fallback)):
        with gc_paused():
            ramp_clock(torch, fn, seconds=0.1)
            eager = time_launches(torch, fn, steps, warmup)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(3):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn(0)
        with gc_paused():  # the capture idled the GPU: ramp its clock again first
            ramp_clock(torch, lambda i: graph.replay(), seconds=0.1)
            replay = time_launches(torch, lambda i: graph.replay(), steps, warmup)
        res[name] = {"eager_ms": round(eager, 5), "graph_ms": round(replay, 5)}
    torch.cuda.synchronize()
    # the two compute the same gradients (fp16 GEMM outputs in the fallback)
    rel = max(float((dws[i] - out_t[f"dw{i + 1}"]).norm() / dws[i].norm()) for i in range(3))
    res["max_rel_frobenius_difference"] = round(rel, 5)
    return res


def load_traffic(workload):
    """HBM bytes per launch of the workload's kernel, from the calibrated
    rocprofv3 FETCH_SIZE + WRITE_SIZE runs recorded in profiles/traffic.json
    (None when that workload has not been profiled)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get(workload)
    except (OSError, ValueError):
        return None
    return entry.get("bytes") if isinstance(entry, dict) else None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", choices=sorted(CONFIG_DIMS), default="3l128")
    ap.add_argument("--m", type=int, default=None)
    ap.add_argument("--no-extra", action="store_true",
                    help="headline only: skip the other BASELINE configs, the sweep and the training step")
    ap.add_argument("--train", action="store_true",
                    help="add the longer training experiments (5-layer step, bf16, stash vs recompute, "
                         "the reference's PyTorch-op backward)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--cpu-budget", type=float, default=20.0,
                    help="seconds after which the CPU legs stop repeating (each still runs at least 3 passes)")
    ap.add_argument("--quick", action="store_true",
                    help="counter-collection runs: parity gate, warm-up and the timed launches only (no clock ramp, "
                         "sustained run, bf16 figure or copy reference)")
    ap.add_argument("--train-step", type=int, default=None, metavar="M",
                    help="counter-collection runs of the training kernels: only the WN training step at M rows "
                         "(3 layers; 5 with --config 5l128; no headline, no other legs); prints its timing JSON")
    ap.add_argument("--fwd-step", type=int, default=None, metavar="M",
                    help="counter-collection runs of one forward config: only the forward of --config at M rows "
                         "(element type --fwd-dtype; buffers rotated as for the other configs); prints its JSON")
    ap.add_argument("--fwd-dtype", choices=("fp16", "bf16", "fp32"), default="fp16",
                    help="with --fwd-step: the tensors' element type")
    ap.add_argument("--train-dtype", choices=("fp16", "bf16", "fp32"), default="fp16",
                    help="with --train-step: x's type (fp32 runs the fp32-tensor kernels)")
    ap.add_argument("--train-hidden", type=int, default=128,
                    help="with --train-step: the hidden width H (256: the streamed-weight kernels)")
    ap.add_argument("--sweep", action="store_true",
                    help="only the small-batch latency sweep of --config (M = 64 .. 4096; kernel-trace runs); "
                         "prints its JSON")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py: this build measures ONE GPU; the forward shards rows with zero exchange and "
            "no multi-GPU figure is produced (run with --gpus 1)",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch
    import _mlpmk  # noqa: F401
    from mlpmk import ops
    from oracle import mlp_oracle as orc

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    if args.sweep:
        with gc_paused():
            print(json.dumps({"latency_sweep": latency_sweep(torch, ops, CONFIG_DIMS[args.config]),
                              "config": args.config}))
        return

    if args.fwd_step:
        fdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[args.fwd_dtype]
        with gc_paused():
            r = fwd_bench(torch, ops, CONFIG_DIMS[args.config], args.fwd_step, args.config == "narrow",
                          steps=args.steps, warmup=args.warmup, dtype=fdt)
        print(json.dumps({"forward": {f"{args.config} {args.fwd_dtype} M={args.fwd_step}": r}}))
        return

    if args.train_step:
        n_layers = 5 if args.config == "5l128" else 3
        tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[args.train_dtype]
        print(json.dumps({"training_step": {str(args.train_step): train_step_bench(
            torch, args.train_step, steps=args.steps, warmup=args.warmup, n_layers=n_layers, dtype=tdt,
            hidden=args.train_hidden)}, "layers": n_layers}))
        return

    dims = CONFIG_DIMS[args.config]
    uniform = args.config == "narrow"
    m = args.m or DEFAULT_M[args.config]
    workload = f"{args.config} fwd fp16 M={m}"

    # --- inputs resident in HBM: two buffer pairs rotate -------------------
    x0, ws = make_device_inputs(torch, dims, m, seed=0, uniform=uniform)
    x1, _ = make_device_inputs(torch, dims, m, seed=1, uniform=uniform)
    xs = [x0, x1]
    outs = [torch.empty((m, dims[-1]), device="cuda", dtype=torch.float16) for _ in range(2)]

    def step(i):
        ops.fwd_into(xs[i & 1], ws, outs[i & 1])

    # --- parity gate (sampled rows vs the CPU oracle) ----------------------
    step(0)
    torch.cuda.synchronize()
    idx = torch.randperm(m, device="cuda")[:4096]
    ok, maxerr, _ = orc.allclose_report(
        outs[0][idx].float().cpu().numpy(),
        orc.forward(x0[idx].cpu().numpy(), [w.cpu().numpy() for w in ws]),
        1e-2,
        1e-2,
    )

    # --- timed region: the K launches of the contract ----------------------
    with gc_paused():
        if not args.quick:
            ramp_clock(torch, step)
        ms = time_launches(torch, step, args.steps, args.warmup)
    # the same launches sustained for >= 0.5 s, right after
    sus_ms, sus_n = sustained(torch, step, ms) if not args.quick else (float("nan"), 0)
    nbytes, nflops = algorithmic(dims, m)
    achieved_gbs = nbytes / (ms * 1e-3) / 1e9
    tflops = nflops / (ms * 1e-3) / 1e12
    ai = nflops / nbytes
    roof_tflops = min(MFMA_F16_PEAK_TFLOPS, HBM_PEAK_GBS * ai / 1e3)
    bound = "hbm" if HBM_PEAK_GBS * ai / 1e3 < MFMA_F16_PEAK_TFLOPS else "mfma"

    def frac_of(t_ms):
        if bound == "hbm":
            return nbytes / (t_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
        return nflops / (t_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS

    if bound == "hbm":
        roofline = {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(frac_of(ms), 4)}
    else:
        roofline = {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(frac_of(ms), 4)}
    roofline["traffic"] = load_traffic(workload)
    roofline["kernel"] = "mlpmk::fwd_kernel"
    roofline["algorithmic_bytes_per_launch"] = nbytes
    roofline["timed_over"] = f"the {args.steps} timed launches (HIP events); 'sustained' has the >= 0.5 s figure"

    bf16_ms = copy_gbs = float("nan")
    if args.quick:
        # counter runs: a few copies of known size to calibrate FETCH_SIZE /
        # WRITE_SIZE against (no timing)
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            ops.copy_bytes(src, dst)
        torch.cuda.synchronize()
        del src, dst
    else:
        # The same workload with bf16 tensors (the bf16 instantiation of the
        # kernel; a secondary figure, the metric stays the fp16 one).
        xb = [x.to(torch.bfloat16) for x in xs]
        wb = [w.to(torch.bfloat16) for w in ws]
        ob = [torch.empty_like(o, dtype=torch.bfloat16) for o in outs]
        with gc_paused():
            ramp_clock(torch, lambda i: ops.fwd_into(xb[i & 1], wb, ob[i & 1]))
            bf16_ms = time_launches(torch, lambda i: ops.fwd_into(xb[i & 1], wb, ob[i & 1]), args.steps, args.warmup)
        del xb, wb, ob

        # achievable-HBM reference: the library's 16-byte copy over 512 MiB
        # with the forward's cache policy (default loads, non-temporal
        # stores); 512 MiB each way so that the source cannot stay in the
        # 256 MB Infinity Cache between launches
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        with gc_paused():
            ramp_clock(torch, lambda i: ops.copy_bytes(src, dst), 0.05)
            cms = time_launches(torch, lambda i: ops.copy_bytes(src, dst), 20, 5)
        copy_gbs = 2 * src.numel() / (cms * 1e-3) / 1e9
        del src, dst

    result = {
        "metric": METRIC,
        "value": m / (ms * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) x, N(0,1/in) fp16 weights, resident in HBM)",
        "config": {"workload": workload, "dims": list(dims), "M": m, "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "sustained": None if args.quick else {
            "ms_per_step": round(sus_ms, 5), "launches": sus_n, "seconds": round(sus_ms * sus_n / 1e3, 3),
            "roofline_frac": round(frac_of(sus_ms), 4)},
        "tflops": round(tflops, 2),
        "roofline_tflops": round(roof_tflops, 1),
        "frac_of_min_mfma_hbm_roofline": round(tflops / roof_tflops, 4),
        "copy_kernel_gbs": None if args.quick else round(copy_gbs, 1),
        "copy_kernel": "512 MiB each way, 16-byte default loads + non-temporal stores (the forward's policy), "
                       "3 workgroups of 256 threads per CU (the fastest grid-stride shape measured)",
        "bf16_ms_per_step": None if args.quick else round(bf16_ms, 5),
        "parity": {"ok": ok, "max_abs_err": maxerr, "atol": 1e-2, "rtol": 1e-2, "rows_checked": 4096},
        "device": torch.cuda.get_device_properties(0).name,
        "launch": ops.fwd_launch_info(dims, m),
    }
    if os.environ.get("MLPMK_LIBRARY"):
        result["library"] = os.path.basename(os.environ["MLPMK_LIBRARY"])

    if not args.no_extra:
        # The other BASELINE configs, each timed here too.
        result["configs"] = {
            "3l128 M=65536": fwd_bench(torch, ops, CONFIG_DIMS["3l128"], 65536, False),
            "5l128 M=65536": fwd_bench(torch, ops, CONFIG_DIMS["5l128"], 65536, False),
            "5l128 M=1048576": fwd_bench(torch, ops, CONFIG_DIMS["5l128"], 1048576, False),
            "narrow M=4194304": fwd_bench(torch, ops, CONFIG_DIMS["narrow"], 4194304, True),
            # fp32 tensors (bf16 hi/lo split operands, fp32 rows: twice the bytes)
            "3l128 fp32 M=1048576": fwd_bench(torch, ops, CONFIG_DIMS["3l128"], 1048576, False, dtype=torch.float32),
            # hidden width 256: weights streamed through LDS (fwd_wide.hip)
            "3l256 M=1048576": fwd_bench(torch, ops, CONFIG_DIMS["3l256"], 1048576, False),
        }
        result["latency_sweep"] = latency_sweep(torch, ops, CONFIG_DIMS["3l128"])
        result["training"] = {str(mt): train_step_bench(torch, mt) for mt in (4096, 16384, 131072)}
        # fp32 tensors (bf16 hi/lo split operands) and hidden width 256 (the
        # two-pass backward at every M), same step
        result["training_fp32"] = {str(mt): train_step_bench(torch, mt, steps=20, warmup=5, dtype=torch.float32)
                                   for mt in (4096, 131072)}
        result["training_h256"] = {str(mt): train_step_bench(torch, mt, steps=20, warmup=5, hidden=256)
                                   for mt in (4096, 131072)}

    if args.train:
        result["training_5l"] = {str(mt): train_step_bench(torch, mt, n_layers=5) for mt in (65536, 131072)}
        result["training_bf16"] = {str(mt): train_step_bench(torch, mt, steps=20, warmup=5, dtype=torch.bfloat16)
                                   for mt in (16384, 131072)}
        result["training_stash_vs_recompute"] = {
            str(mt): {pol: train_step_bench(torch, mt, steps=20, warmup=5, recompute=pol) for pol in ("never", "always")}
            for mt in (131072, 1048576)}
        result["training_stash_vs_recompute_5l"] = {
            str(mt): {pol: train_step_bench(torch, mt, steps=20, warmup=5, n_layers=5, recompute=pol)
                      for pol in ("never", "always")}
            for mt in (131072, 1048576)}
        result["backward_vs_pytorch_fallback"] = {str(mt): backward_comparison(torch, ops, mt)
                                                  for mt in (4096, 32768, 131072, 1048576)}

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_eager_baseline(torch, x0, ws, budget_s=args.cpu_budget)
        result["cpu_oracle_numpy"] = cpu_oracle_numpy(orc, x0.cpu().numpy(), [w.cpu().numpy() for w in ws],
                                                      budget_s=args.cpu_budget / 2)
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
