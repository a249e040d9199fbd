"""Benchmark of the MI355X scan on the reference's headline workload.

Default (what the driver runs): ``python bench.py`` -> one GPU, workload C4 of the
reference's north star: pscan forward + backward on (batch 8, dim 1024, seqlen 65536) bf16,
synthetic Mamba-style inputs (gates = exp(-softplus(N(0,1)) * U[0.001, 0.1]),
tokens = 0.1 N(0,1), grad_out = N(0,1)), resident in HBM before timing starts.

One step = ``pscan(gates, tokens)`` + ``torch.autograd.grad`` of it with ``grad_out``: the
forward kernel and the fused backward kernel. Algorithmic bytes per step, N = B*D*L and s =
itemsize (eval/benchmark.py:62-65 counts the forward the same way):
    forward  3*N*s  (read gates, tokens; write out)
    backward 5*N*s  (read gates, out, grad_out; write grad_gates, grad_tokens)
    step     8*N*s
``value`` = step bytes / (bracketed wall time of K steps / K), in GB/s. ``roofline`` is the
backward kernel (the dominant one), timed alone on the stream it runs on and on the timed
step's own buffers: K back-to-back calls inside one HIP event pair, 5*N*s bytes over the mean
duration.
``cpu_baseline`` times the reference's CPU path -- Hillis-Steele ``parallel_scan_torch``
forward plus the PScan.backward composition -- on a bounded sample of rows of the same
inputs, on the host cores.

Beside the headline, the default line also carries ``rows_f``: the fused softplus-gate scan,
the channel-last scan and ``dimwise_forward`` at the same shape in bf16 (``--no-rows`` skips
them); ``share_b1``: one GPU's share when the batch is split over eight (B1 D1024 L65536, bf16
and fp32, forward and backward, with a roofline block); ``c2``: the reference's published
benchmark (fp32 B2 D256, seqlen 32..65536, forward and reverse) beside the reference's own
p50s; ``c3`` and ``c5``: configs 3 and 5 of WORKLOADS (``--no-configs`` skips these four).

Other workloads (``--workload``), for measurement runs: c1, c2 (fp32 seqlen sweep, forward
and reverse), c3, c5 (plus its (batch, seqlen, dim) .mT variant), c4cl and c5cl (channel-last),
dw (dimwise_forward, beside the copy of its access pattern), c4fused (fused softplus gates),
ceiling (the library's copy probes with the scans' access patterns, beside the scans, row and
channel-last), share (the B1 share object alone) and rows (the row scans on any
``--shape batch,dim,seqlen``; with ``--tiling 1`` or ``2`` it measures either path). Multi-GPU runs are not part of this
build: ``--gpus N`` with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published peak

DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
SHORT = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}

# workload -> (batch, dim, seqlen, dtype, input distribution)
WORKLOADS = {
    "c1": (2, 256, 1024, "float32", "uniform"),
    "c3": (4, 512, 8192, "bfloat16", "uniform"),
    "c4": (8, 1024, 65536, "bfloat16", "mamba"),
    "c5": (64, 4096, 256, "float32", "sigmoid"),
}
C2_SEQLENS = [2 ** k for k in range(5, 17)]
METRIC = "fwd+bwd scan GB/s and % HBM peak; p50 ms at B8 D1024 L65536 bf16"


def make_inputs(batch, dim, seqlen, dtype, dist, seed=0, device="cuda", grad=True):
    """Seeded synthetic inputs of one workload: (gates, tokens, grad_out or None), contiguous
    (batch, dim, seqlen) tensors of ``dtype``, drawn in fp32 then rounded."""
    gen = torch.Generator(device=device).manual_seed(seed)
    shape = (batch, dim, seqlen)

    def rand():
        return torch.rand(shape, generator=gen, device=device)

    def randn():
        return torch.randn(shape, generator=gen, device=device)

    if dist == "uniform":  # configs 1-3
        gates = 0.99 + 0.01 * rand()
        tokens = randn() / seqlen
    elif dist == "mamba":  # config 4
        dt = 0.001 + 0.099 * rand()
        gates = torch.exp(-torch.nn.functional.softplus(randn()) * dt)
        del dt
        tokens = 0.1 * randn()
    elif dist == "sigmoid":  # config 5
        gates = torch.sigmoid(2.0 + randn())
        tokens = randn()
    else:
        raise ValueError(dist)
    grad_out = randn().to(dtype).contiguous() if grad else None
    return gates.to(dtype).contiguous(), tokens.to(dtype).contiguous(), grad_out


# ------------------------------------------------------------------------------ timing
def _events(n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def time_each(fn, warmup, iters, before=None):
    """Per-call durations (ms) from HIP event pairs on the current stream (the stream every
    fpscan kernel is launched on). `before`, if given, runs ahead of each call, outside the
    events (a cache flush). The garbage collector is paused meanwhile: a collection between
    an event and the launch after it would count as kernel time."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts, ends = _events(iters), _events(iters)
    gc_was_on = gc.isenabled()
    gc.disable()
    try:
        for i in range(iters):
            if before is not None:
                before()
            starts[i].record()
            fn()
            ends[i].record()
        torch.cuda.synchronize()
    finally:
        if gc_was_on:
            gc.enable()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def time_bracketed(fn, warmup, iters):
    """Mean duration (ms) of `iters` back-to-back calls: one HIP event pair on the current
    stream around the whole timed region, as the headline step is timed. Unlike per-call event
    pairs it adds no event between the calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = _events(2)
    gc_was_on = gc.isenabled()
    gc.disable()
    try:
        start.record()
        for _ in range(iters):
            fn()
        end.record()
        torch.cuda.synchronize()
    finally:
        if gc_was_on:
            gc.enable()
    return start.elapsed_time(end) / iters


def cache_flusher(mib=1024):
    """A callable that writes `mib` MiB (4x the 256 MB MALL, 32x the 32 MB of L2) so that the
    next kernel finds none of its operands cached."""
    buf = torch.empty(mib << 18, dtype=torch.float32, device="cuda")
    state = {"v": 0.0}

    def flush():
        state["v"] += 1.0
        buf.fill_(state["v"])

    return flush


def percentile(xs, q):
    s = sorted(xs)
    if not s:
        return float("nan")
    k = (len(s) - 1) * q
    lo, hi = math.floor(k), math.ceil(k)
    return s[lo] + (s[hi] - s[lo]) * (k - lo)


# ------------------------------------------------------------------------------ CPU baseline
def cpu_baseline(gates, tokens, grad_out, target_s):
    """Reference CPU path (Hillis-Steele forward + PScan.backward composition with the
    Hillis-Steele reverse scan) on the first rows of the inputs, sized to about target_s."""
    import oracle  # the cpu_baseline leg is the one place bench.py uses the oracle package

    torch.set_num_threads(os.cpu_count() or 1)
    B, D, L = gates.shape
    rows_total = B * D
    s = gates.element_size()

    def run(rows):
        g = gates.reshape(rows_total, L)[:rows].cpu()
        x = tokens.reshape(rows_total, L)[:rows].cpu()
        go = grad_out.reshape(rows_total, L)[:rows].cpu()
        t0 = time.perf_counter()
        y = oracle.parallel_scan_torch(g, x)
        oracle.pscan_backward_composed(g, y, go, oracle.parallel_scan_torch)
        return time.perf_counter() - t0

    rows = 1
    dt = run(rows)
    while dt < 0.5 and rows < rows_total:  # grow until one run is measurable
        rows = min(rows_total, rows * 4)
        dt = run(rows)
    rows = max(1, min(rows_total, int(rows * max(1.0, target_s / 3 / max(dt, 1e-6)))))
    times = [run(rows) for _ in range(3)]
    p50 = statistics.median(times)
    gbps = 8 * rows * L * s / p50 / 1e9
    return {
        "value": round(gbps, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{rows} of {rows_total} rows x {L} {SHORT[gates.dtype]}: Hillis-Steele "
                  f"forward + composed backward (eval/baselines.py:40-61, fpscan/ops.py:69-83), "
                  f"p50 of 3 runs ({p50:.2f} s each)",
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def _cpu_model():
    """The host CPU's model string from /proc/cpuinfo (platform.processor() only says
    'x86_64' on Linux)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline_c1(warmup=3, iters=20):
    """Config 1 (fp32 B2 D256 L1024) on the host cores: the reference's CPU path (Hillis-Steele
    ``parallel_scan_torch`` forward, eval/baselines.py:40-61) on fp32 B2 D256 L1024 with the
    reference test's distributions, warmup 3 then p50 of 20 (GB/s at 3*N*4 bytes)."""
    import oracle  # the cpu_baseline leg

    torch.set_num_threads(os.cpu_count() or 1)
    B, D, L = WORKLOADS["c1"][:3]
    gen = torch.Generator().manual_seed(0)
    g = 0.99 + 0.01 * torch.rand(B, D, L, generator=gen)
    x = torch.randn(B, D, L, generator=gen) / L
    for _ in range(warmup):
        oracle.parallel_scan_torch(g, x)
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        oracle.parallel_scan_torch(g, x)
        times.append(time.perf_counter() - t0)
    p50 = statistics.median(times)
    return {
        "value": round(3 * B * D * L * 4 / p50 / 1e9, 4),
        "unit": "GB/s",
        "p50_ms": round(p50 * 1e3, 4),
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"config 1: fp32 B{B} D{D} L{L} Hillis-Steele forward (eval/baselines.py:40-61),"
                  f" warmup {warmup}, p50 of {iters}",
        "cpu_model": _cpu_model(),
    }


def load_traffic(workload, dtype_short):
    """HBM bytes per backward launch measured by rocprofv3 PMC counters (FETCH_SIZE,
    WRITE_SIZE, scaled by a copy kernel of known size), committed under profiles/."""
    rel = os.path.join("profiles", f"pmc_traffic_{workload}_{dtype_short}.json")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), rel)
    try:
        with open(path) as f:
            d = json.load(f)
        return d.get("bwd_bytes_per_launch"), rel  # relative to the repository root
    except (OSError, ValueError):
        return None, None


# ------------------------------------------------------------------------------ workloads
def measure_training_step(B, D, L, dtype, dist, steps, warmup, workload):
    """One dtype of the headline workload: K bracketed fwd+bwd steps, their per-step p50/p90,
    and each kernel timed alone (HIP events on the stream the kernels run on). Returns the
    figures and the inputs (for the CPU baseline)."""
    import fpscan_amd

    N = B * D * L
    s = torch.empty((), dtype=dtype).element_size()
    gates, tokens, grad_out = make_inputs(B, D, L, dtype, dist, seed=0)
    g = gates.clone().requires_grad_()
    x = tokens.clone().requires_grad_()

    def step():
        out = fpscan_amd.pscan(g, x)
        return torch.autograd.grad(out, (g, x), grad_out)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # K timed steps, bracketed by a synchronisation on both sides (one process, one GPU); the
    # garbage collector is paused, as in time_each
    start, end = _events(2)
    gc.disable()
    try:
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            step()
        end.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3
    finally:
        gc.enable()
    ms_per_step = start.elapsed_time(end) / steps
    step_p = time_each(step, 1, steps)

    # Kernels alone, on the timed step's own buffers: its inputs, and the forward output and
    # the two gradients of one more step (the caching allocator hands every step the same
    # blocks). The kernels' speed depends on where their tensors sit in HBM by several per
    # cent (the fused backward at the headline: 842-871 us over six output placements in one
    # process), so buffers allocated apart from the step would time a different placement.
    y = fpscan_amd.pscan(g, x)
    gg, gx = torch.autograd.grad(y, (g, x), grad_out)
    y = y.detach()
    gd, xd = g.detach(), x.detach()
    fwd = lambda: fpscan_amd.scan_forward(gd, xd, out=y)  # noqa: E731
    fwd_t = time_each(fwd, 2, steps)
    bwd = lambda: fpscan_amd.scan_backward(gd, y, grad_out, gg, gx)  # noqa: E731
    bwd_t = time_each(bwd, 2, steps)
    # the roofline's average launch duration: one event pair over `steps` back-to-back calls
    fwd_avg = time_bracketed(fwd, 2, steps)
    bwd_avg = time_bracketed(bwd, 2, steps)
    del y, gg, gx, gd, xd, g, x
    bwd_bytes = 5 * N * s
    achieved = bwd_bytes / (bwd_avg / 1e3) / 1e9
    traffic, traffic_src = load_traffic(workload, SHORT[dtype])
    value = 8 * N * s / (ms_per_step / 1e3) / 1e9
    dcode = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    tiled = fpscan_amd.ops._load_extension().workspace_bytes(B, D, L, dcode, 1) > 0
    bwd_kernel = ("scan_tiles<bwd> (fused backward, persistent tiles with look-back)" if tiled
                  else "scan_long_rows<bwd> (fused backward, one block per row)")
    res = {
        "value": round(value, 2),
        "ms_per_step": round(ms_per_step, 5),
        "p50_ms": round(percentile(step_p, 0.5), 5),
        "p90_ms": round(percentile(step_p, 0.9), 5),
        "hbm_frac": round(value / HBM_PEAK_GBPS, 4),
        "fwd_kernel": {"avg_ms": round(fwd_avg, 5), "p50_ms": round(percentile(fwd_t, 0.5), 5),
                       "gbps": round(3 * N * s / (fwd_avg / 1e3) / 1e9, 1)},
        "bwd_kernel": {"avg_ms": round(bwd_avg, 5), "p50_ms": round(percentile(bwd_t, 0.5), 5),
                       "gbps": round(achieved, 1)},
        "kernel_timing": "on the timed step's own buffers; avg_ms: one event pair over "
                         "back-to-back calls (the roofline's average launch duration); "
                         "p50_ms: per-call event pairs",
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel": bwd_kernel,
            "algorithmic_bytes_per_launch": bwd_bytes,
            "traffic_source": traffic_src,
        },
        "wall_ms_timed_region": round(wall_ms, 3),
    }
    return res, (gates, tokens, grad_out)


# Each workload after the first starts from an empty allocator cache, as it would in a
# process of its own: where a workload's tensors land inside segments cached by an earlier
# workload changes its speed by a few per cent (measured: the fused softplus-gate step 1.503 ms
# in a fresh process, 1.556 ms after the headline's bf16 and fp32 steps, 1.505-1.510 ms after
# releasing the cache). The driver wipes released memory in the background and a measurement
# overlapping that wipe stalls (10-17 ms once in two runs when the release came right before
# it), so the release is followed by a pause of RELEASE_PAUSE_S, and each measurement then by
# WARM_CALLS untimed calls: the first few dozen milliseconds of GPU work after a pause run a
# few per cent slow (the channel-last forward's first 20 calls 587 us, then 566-568).
WARM_CALLS = 20
RELEASE_PAUSE_S = 2.0


def fresh_allocator():
    """Returns torch's cached device memory to the driver and waits for it to settle."""
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.synchronize()
    time.sleep(RELEASE_PAUSE_S)


def rows_f_summary(iters):
    """The next-step rows at the headline shape (B8 D1024 L65536 bf16), reported beside the
    headline line so that each has a driver-measured figure: the fused softplus-gate scan
    (forward and backward kernels alone, and the autograd step), the channel-last scan
    (forward and backward, tensors (8, 65536, 1024), and the first batch alone) and
    dimwise_forward. p50 over `iters` calls; GB/s of algorithmic bytes (forward 3 N s,
    backward 5 N s, step 8 N s)."""
    import fpscan_amd

    B, D, L = 8, 1024, 65536
    dtype = torch.bfloat16
    s = 2
    N = B * D * L

    def gbps(nbytes, ms):
        return round(nbytes / (ms / 1e3) / 1e9, 1)

    def timed(fn, nbytes, before=None):
        p50 = percentile(time_each(fn, WARM_CALLS, iters, before), 0.5)
        return {"p50_ms": round(p50, 5), "gbps": gbps(nbytes, p50),
                "hbm_frac": round(gbps(nbytes, p50) / HBM_PEAK_GBPS, 4)}

    out = {"shape": "B8 D1024 L65536 bf16", "iters": iters}
    # fused softplus gates: gates = exp(-softplus(z) * rate[d]) computed inside the kernels
    gen = torch.Generator(device="cuda").manual_seed(3)
    z = torch.randn(B, D, L, generator=gen, device="cuda").to(dtype)
    rate = 0.001 + 0.099 * torch.rand(D, generator=gen, device="cuda")
    x = (0.1 * torch.randn(B, D, L, generator=gen, device="cuda")).to(dtype)
    go = torch.randn(B, D, L, generator=gen, device="cuda").to(dtype)
    y = torch.empty_like(x)
    fused = {
        "fwd_kernel": timed(lambda: fpscan_amd.scan_forward_softplus(z, rate, x, out=y),
                            3 * N * s),
        "bwd_kernel": timed(lambda: fpscan_amd.scan_backward_softplus(z, rate, y, go),
                            5 * N * s),
    }
    zr, rr, xr = (t.clone().requires_grad_() for t in (z, rate, x))
    del z, x, y
    fresh_allocator()

    def step():
        return torch.autograd.grad(fpscan_amd.pscan_softplus(zr, rr, xr), (zr, rr, xr), go)

    fused["step"] = timed(step, 8 * N * s)
    out["softplus_fused"] = fused
    del rate, go, zr, rr, xr
    fresh_allocator()
    # channel-last (batch, seqlen, dim)
    g, x, go = make_inputs(B, L, D, dtype, "mamba", seed=1)
    y = fpscan_amd.scan_forward_channel_last(g, x)
    o, gg, gx = torch.empty_like(x), torch.empty_like(x), torch.empty_like(x)
    out["channel_last"] = {
        "fwd": timed(lambda: fpscan_amd.scan_forward_channel_last(g, x, False, o), 3 * N * s),
        "bwd": timed(lambda: fpscan_amd.scan_backward_channel_last(g, y, go, gg, gx), 5 * N * s),
    }
    # the same at batch 1 (16 chains of 64 columns: one GPU's share when the batch is split
    # over eight), which takes the wide look-back; GB/s of that batch's bytes
    g1, x1, go1, y1, o1, gg1, gx1 = (t[:1] for t in (g, x, go, y, o, gg, gx))
    n1 = N // B
    out["channel_last_batch1"] = {
        "fwd": timed(lambda: fpscan_amd.scan_forward_channel_last(g1, x1, False, o1),
                     3 * n1 * s),
        "bwd": timed(lambda: fpscan_amd.scan_backward_channel_last(g1, y1, go1, gg1, gx1),
                     5 * n1 * s),
    }
    del g, x, go, y, o, gg, gx, g1, x1, go1, y1, o1, gg1, gx1
    fresh_allocator()
    # dimwise_forward, in place on Bx, restored from the same input before each timed call
    # (outside the events; see bench_dimwise)
    G = fpscan_amd.dimwise_groups(L)
    gen = torch.Generator(device="cuda").manual_seed(2)
    ax = (0.99 + 0.01 * torch.rand(B, D, L, generator=gen, device="cuda")).to(dtype)
    bx0 = (torch.randn(B, D, L, generator=gen, device="cuda") / G).to(dtype)
    bh = (torch.randn(B, D, G, generator=gen, device="cuda") / G).to(dtype)
    wq = (0.01 * torch.rand(D, generator=gen, device="cuda")).to(dtype)
    wk = (0.01 * torch.rand(D, generator=gen, device="cuda")).to(dtype)
    bx = bx0.clone()
    out["dimwise"] = timed(lambda: fpscan_amd.dimwise_forward(ax, bx, bh, wq, wk), 3 * N * s,
                           before=lambda: bx.copy_(bx0))
    del ax, bx0, bx, bh, wq, wk
    return out


# The reference's published table (README.md:47-60; eval/benchmark.py:132-217): fp32 B2 D256
# forward scan_forward on an NVIDIA GeForce RTX 4060 Laptop GPU, p50 ms over 100 iterations.
REF_C2_P50_MS = {32: 0.0074, 64: 0.0079, 128: 0.0073, 256: 0.0081, 512: 0.0075, 1024: 0.0092,
                 2048: 0.0133, 4096: 0.0328, 8192: 0.2008, 16384: 0.4362, 32768: 0.8612,
                 65536: 1.7050}


def _timed_entry(fn, nbytes, iters, warm=WARM_CALLS):
    """p50/p90 (ms) over `iters` calls timed with an event pair each, after `warm` untimed
    ones, their mean, and GB/s and fraction of peak at the p50."""
    t = time_each(fn, warm, iters)
    p50 = percentile(t, 0.5)
    gbps = nbytes / (p50 / 1e3) / 1e9
    return {"p50_ms": round(p50, 5), "p90_ms": round(percentile(t, 0.9), 5),
            "avg_ms": round(statistics.mean(t), 5), "gbps": round(gbps, 1),
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)}


def share_summary(iters):
    """One GPU's share of the headline when its batch is split over eight GPUs: B1 D1024
    L65536 (1024 rows of 65536, the few-rows regime the reference handles with one block per
    row, full_scan.cu:77-80, 190), in bf16 and fp32. Forward and fused backward kernels alone,
    each on the path the library picks for the size, with a roofline block for the backward
    (the larger kernel): 5 N s bytes over its mean event-timed duration."""
    import fpscan_amd

    B, D, L = 1, 1024, 65536
    ext = fpscan_amd.ops._load_extension()
    res = {"shape": f"B{B} D{D} L{L}", "iters": iters}
    for dtype in (torch.bfloat16, torch.float32):
        s = torch.empty((), dtype=dtype).element_size()
        N = B * D * L
        gates, tokens, grad_out = make_inputs(B, D, L, dtype, "mamba", seed=4)
        out = torch.empty_like(tokens)
        y = fpscan_amd.scan_forward(gates, tokens)
        gg, gx = torch.empty_like(gates), torch.empty_like(gates)
        dcode = {torch.float32: 0, torch.bfloat16: 2}[dtype]
        paths = {op: ("scan_tiles" if ext.workspace_bytes(B, D, L, dcode, k) > 0
                      else "scan_long_rows") for k, op in ((0, "fwd"), (1, "bwd"))}
        fwd_fn = lambda: fpscan_amd.scan_forward(gates, tokens, False, out)  # noqa: E731
        bwd_fn = lambda: fpscan_amd.scan_backward(gates, y, grad_out, gg, gx)  # noqa: E731
        fwd = _timed_entry(fwd_fn, 3 * N * s, iters)
        bwd = _timed_entry(bwd_fn, 5 * N * s, iters)
        # the roofline's average launch duration: one event pair over back-to-back calls
        fwd["avg_ms"] = round(time_bracketed(fwd_fn, 2, iters), 5)
        bwd["avg_ms"] = round(time_bracketed(bwd_fn, 2, iters), 5)
        achieved = 5 * N * s / (bwd["avg_ms"] / 1e3) / 1e9
        traffic, src = load_traffic("share_b1", SHORT[dtype])
        res[SHORT[dtype]] = {
            "paths": paths, "fwd": fwd, "bwd": bwd,
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                         "traffic": traffic, "kernel": f"{paths['bwd']}<bwd>",
                         "algorithmic_bytes_per_launch": 5 * N * s, "traffic_source": src},
        }
        del gates, tokens, grad_out, out, y, gg, gx
    return res


def c2_summary(iters, warmup=10):
    """Config 2, the reference's only published benchmark: fp32 B2 D256 scan_forward over
    seqlen 32..65536 with eval/benchmark.py's inputs and call (a fresh output per call), warmup
    10 and p50/p90 over `iters`, forward and reverse. Each forward point carries the reference's
    published p50 (README.md:47-60, an RTX 4060 Laptop GPU) and the ratio to it."""
    import fpscan_amd

    rows = []
    for L in C2_SEQLENS:
        gates, tokens, _ = make_inputs(2, 256, L, torch.float32, "uniform", seed=L, grad=False)
        nbytes = 3 * 2 * 256 * L * 4
        row = {"seqlen": L}
        for name, rev in (("fwd", False), ("rev", True)):
            t = time_each(lambda: fpscan_amd.scan_forward(gates, tokens, rev), warmup, iters)
            p50 = percentile(t, 0.5)
            row[name] = {"p50_ms": round(p50, 5), "p90_ms": round(percentile(t, 0.9), 5),
                         "gbps": round(nbytes / (p50 / 1e3) / 1e9, 1)}
        row["ref_fwd_p50_ms"] = REF_C2_P50_MS[L]
        row["speedup_vs_ref"] = round(REF_C2_P50_MS[L] / row["fwd"]["p50_ms"], 2)
        rows.append(row)
        del gates, tokens
    # What the same timing reads with no scan: an event pair around a call that launches no
    # kernel (the output allocation alone), and around torch's own smallest kernel at the
    # seqlen-32 shape. At short seqlens a scan call costs about what the latter does.
    x = torch.zeros((2, 256, 32), dtype=torch.float32, device="cuda")
    alloc = time_each(lambda: torch.empty_like(x), warmup, iters)
    add = time_each(lambda: x.add_(0.0), warmup, iters)
    floor = {"alloc_only_p50_ms": round(percentile(alloc, 0.5), 5),
             "torch_add_p50_ms": round(percentile(add, 0.5), 5)}
    return {"shape": "fp32 B2 D256", "iters": iters, "warmup": warmup,
            "ref_source": "README.md:47-60 (RTX 4060 Laptop GPU, fp32 forward)", "rows": rows,
            "event_floor_l32": floor}


def c3_summary(iters):
    """Config 3: bf16 and fp16 B4 D512 L8192 (fp32 accumulation), forward, reverse and fused
    backward kernels alone, and the autograd step (pscan + torch.autograd.grad)."""
    import fpscan_amd

    B, D, L = WORKLOADS["c3"][:3]
    N = B * D * L
    res = {"shape": f"B{B} D{D} L{L}", "iters": iters}
    for dtype in (torch.bfloat16, torch.float16):
        s = torch.empty((), dtype=dtype).element_size()
        gates, tokens, grad_out = make_inputs(B, D, L, dtype, "uniform", seed=1)
        out = torch.empty_like(tokens)
        y = fpscan_amd.scan_forward(gates, tokens)
        gg, gx = torch.empty_like(gates), torch.empty_like(gates)
        g = gates.clone().requires_grad_()
        x = tokens.clone().requires_grad_()

        def step():
            return torch.autograd.grad(fpscan_amd.pscan(g, x), (g, x), grad_out)

        res[SHORT[dtype]] = {
            "fwd": _timed_entry(lambda: fpscan_amd.scan_forward(gates, tokens, False, out),
                                3 * N * s, iters),
            "rev": _timed_entry(lambda: fpscan_amd.scan_forward(gates, tokens, True, out),
                                3 * N * s, iters),
            "bwd": _timed_entry(lambda: fpscan_amd.scan_backward(gates, y, grad_out, gg, gx),
                                5 * N * s, iters),
            "step": _timed_entry(step, 8 * N * s, iters),
        }
        del gates, tokens, grad_out, out, y, gg, gx, g, x
    return res


def c5_summary(iters):
    """Config 5: fp32 B64 D4096 L256 (many short rows), forward, reverse and backward kernels
    alone, and the same data held as (batch, seqlen, dim): transposed in with .mT.contiguous(),
    scanned and transposed back (README.md:94-99), timed end to end."""
    import fpscan_amd

    B, D, L = WORKLOADS["c5"][:3]
    N = B * D * L
    s = 4
    gates, tokens, grad_out = make_inputs(B, D, L, torch.float32, "sigmoid", seed=1)
    out = torch.empty_like(tokens)
    y = fpscan_amd.scan_forward(gates, tokens)
    gg, gx = torch.empty_like(gates), torch.empty_like(gates)
    res = {"shape": f"B{B} D{D} L{L} f32", "iters": iters,
           "fwd": _timed_entry(lambda: fpscan_amd.scan_forward(gates, tokens, False, out),
                               3 * N * s, iters),
           "rev": _timed_entry(lambda: fpscan_amd.scan_forward(gates, tokens, True, out),
                               3 * N * s, iters),
           "bwd": _timed_entry(lambda: fpscan_amd.scan_backward(gates, y, grad_out, gg, gx),
                               5 * N * s, iters)}
    del out, y, gg, gx, grad_out
    gt, xt = gates.mT.contiguous(), tokens.mT.contiguous()
    del gates, tokens

    def e2e():
        return fpscan_amd.scan_forward(gt.mT.contiguous(), xt.mT.contiguous()).mT.contiguous()

    # scan bytes only (3 N s): the three transposes add 6 N s of copies on top
    res["fwd_via_mT"] = _timed_entry(e2e, 3 * N * s, iters)
    del gt, xt
    return res


def bench_headline(args):
    B, D, L, dname, dist = WORKLOADS[args.workload]
    dtype = DTYPES[args.dtype or dname]
    main, inputs = measure_training_step(B, D, L, dtype, dist, args.steps, args.warmup,
                                         args.workload)
    res = {
        "metric": METRIC,
        "value": main.pop("value"),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": SHORT[dtype],
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: pscan fwd+bwd B{B} D{D} L{L} {SHORT[dtype]}",
            "batch": B, "dim": D, "seqlen": L, "inputs": dist,
            "parallelism": "none (1 GPU; rows independent)",
        },
    }
    res.update(main)
    res["device"] = torch.cuda.get_device_name()
    if args.workload == "c4" and dtype != torch.float32 and not args.no_fp32:
        # the north star's second dtype, fp32 (the reference's only published dtype): the same
        # step at the same shape, reported beside the headline line's bf16 figures
        fresh_allocator()
        f32, _ = measure_training_step(B, D, L, torch.float32, dist, args.steps, args.warmup,
                                       args.workload)
        f32["config"] = f"{args.workload}: pscan fwd+bwd B{B} D{D} L{L} f32"
        res["fp32"] = f32
    if args.workload == "c4" and not args.no_rows:
        fresh_allocator()
        res["rows_f"] = rows_f_summary(args.steps)
    if args.workload == "c4" and not args.no_configs:
        # the one-GPU share of the sharded headline, and configs 2, 3 and 5
        for key, fn, n in (("share_b1", share_summary, args.steps), ("c2", c2_summary, args.iters),
                           ("c3", c3_summary, args.steps), ("c5", c5_summary, args.steps)):
            fresh_allocator()
            res[key] = fn(n)
    # The CPU baselines run last, after every GPU measurement, so that 15 s of host work
    # never sits between two of them.
    if args.no_cpu_baseline:
        res["cpu_baseline"] = None
    else:
        res["cpu_baseline"] = cpu_baseline(*inputs, args.cpu_seconds)
    del inputs
    if not args.no_cpu_baseline:
        res["cpu_baseline_c1"] = cpu_baseline_c1()
    return res


def bench_sweep(args):
    """Config 2: fp32 B2 D256 forward and reverse scan_forward over seqlen 32..65536
    (eval/benchmark.py's table: p50/p90 ms and GB/s = 3*N*s / p50)."""
    import fpscan_amd

    rows = []
    flush = cache_flusher() if args.flush else None
    seqlens = args.seqlens or C2_SEQLENS
    for L in seqlens:
        gates, tokens, _ = make_inputs(2, 256, L, torch.float32, "uniform", seed=L, grad=False)
        out = torch.empty_like(tokens)
        for rev in (False, True):
            t = time_each(lambda: fpscan_amd.scan_forward(gates, tokens, rev, out), 10, args.iters,
                          before=flush)
            p50 = percentile(t, 0.5)
            rows.append({"seqlen": L, "reverse": rev, "p50_ms": round(p50, 5),
                         "p90_ms": round(percentile(t, 0.9), 5),
                         "gbps": round(3 * 2 * 256 * L * 4 / (p50 / 1e3) / 1e9, 1),
                         "caches": "flushed" if args.flush else "warm"})
            print(json.dumps(rows[-1]), flush=True)
    return {"workload": "c2: fp32 B2 D256 forward/reverse sweep", "rows": rows}


def bench_shape(args):
    """c1 / c3 / c5, or rows (any --shape B,D,L; bf16 unless --dtype): forward, reverse and
    backward kernels alone, p50 over --iters. With --tiling 1 or 2, one path (the path
    choice's crossovers are measured this way)."""
    import fpscan_amd

    if args.workload == "rows":
        B, D, L = args.shape
        dname, dist = "bfloat16", "mamba"
    else:
        B, D, L, dname, dist = WORKLOADS[args.workload]
    dtypes = [DTYPES[args.dtype]] if args.dtype else (
        [torch.bfloat16, torch.float16] if args.workload == "c3" else [DTYPES[dname]])
    res = {"workload": args.workload, "shape": [B, D, L], "results": []}
    for dtype in dtypes:
        s = torch.empty((), dtype=dtype).element_size()
        N = B * D * L
        gates, tokens, grad_out = make_inputs(B, D, L, dtype, dist, seed=1)
        out = torch.empty_like(tokens)
        y = fpscan_amd.scan_forward(gates, tokens)
        gg, gx = torch.empty_like(gates), torch.empty_like(gates)
        entry = {"dtype": SHORT[dtype]}
        for name, fn, nbytes in (
            ("fwd", lambda: fpscan_amd.scan_forward(gates, tokens, False, out), 3 * N * s),
            ("rev", lambda: fpscan_amd.scan_forward(gates, tokens, True, out), 3 * N * s),
            ("bwd", lambda: fpscan_amd.scan_backward(gates, y, grad_out, gg, gx), 5 * N * s),
        ):
            t = time_each(fn, WARM_CALLS, args.iters)
            p50 = percentile(t, 0.5)
            entry[name] = {"p50_ms": round(p50, 5), "gbps": round(nbytes / (p50 / 1e3) / 1e9, 1)}
        if args.workload == "c5":
            # (batch, seqlen, dim) data: transpose in, scan, transpose out (README.md:94-99)
            gt = gates.mT.contiguous()
            xt = tokens.mT.contiguous()

            def e2e():
                return fpscan_amd.scan_forward(gt.mT.contiguous(), xt.mT.contiguous()).mT.contiguous()

            t = time_each(e2e, WARM_CALLS, args.iters)
            entry["fwd_via_mT"] = {"p50_ms": round(percentile(t, 0.5), 5)}
        res["results"].append(entry)
        print(json.dumps(entry), flush=True)
    return res


def bench_channel_last(args):
    """c4cl / c5cl: configs 4 and 5 with (batch, seqlen, dim) tensors. Times the channel-last
    kernels (fwd, rev, fused bwd) and, for comparison, the reference's recipe for this layout:
    transpose in, row-major scan, transpose out (README.md:94-99)."""
    import fpscan_amd

    B, D, L, dname, dist = WORKLOADS[args.workload[:2]]
    B = args.batch or B
    dtype = DTYPES[args.dtype or dname]
    s = torch.empty((), dtype=dtype).element_size()
    N = B * D * L
    gr, xr, gor = make_inputs(B, D, L, dtype, dist, seed=1)
    g, x, go = (t.mT.contiguous() for t in (gr, xr, gor))  # (batch, seqlen, dim)
    del gr, xr, gor
    out = torch.empty_like(x)
    y = fpscan_amd.scan_forward_channel_last(g, x)
    gg, gx = torch.empty_like(g), torch.empty_like(g)
    entry = {"workload": args.workload, "shape_bld": [B, L, D], "dtype": SHORT[dtype]}
    for name, fn, nbytes in (
        ("fwd", lambda: fpscan_amd.scan_forward_channel_last(g, x, False, out), 3 * N * s),
        ("rev", lambda: fpscan_amd.scan_forward_channel_last(g, x, True, out), 3 * N * s),
        ("bwd", lambda: fpscan_amd.scan_backward_channel_last(g, y, go, gg, gx), 5 * N * s),
    ):
        t = time_each(fn, WARM_CALLS, args.iters)
        p50 = percentile(t, 0.5)
        entry[name] = {"p50_ms": round(p50, 5), "gbps": round(nbytes / (p50 / 1e3) / 1e9, 1)}

    def via_transpose():
        return fpscan_amd.scan_forward(g.mT.contiguous(), x.mT.contiguous()).mT.contiguous()

    t = time_each(via_transpose, WARM_CALLS, args.iters)
    p50 = percentile(t, 0.5)
    entry["fwd_via_transpose"] = {"p50_ms": round(p50, 5),
                                  "gbps": round(3 * N * s / (p50 / 1e3) / 1e9, 1)}
    print(json.dumps(entry), flush=True)
    return entry


def bench_fused(args):
    """c4fused: the Mamba-style step with the gate producer fused in, at the headline shape.
    Fused: pscan_softplus(z, rate, x) forward + backward (reads z, x, writes y; reads z, y,
    grad_out, writes grad_z, grad_x: 8 N s bytes). Unfused, for comparison: torch computes
    gates = exp(-softplus(z) * rate) and autograd runs pscan and the producer's backward."""
    import fpscan_amd

    B, D, L = 8, 1024, 65536
    dtype = DTYPES[args.dtype or "bfloat16"]
    s = torch.empty((), dtype=dtype).element_size()
    N = B * D * L
    gen = torch.Generator(device="cuda").manual_seed(3)
    z = torch.randn(B, D, L, generator=gen, device="cuda").to(dtype).requires_grad_()
    rate = (0.001 + 0.099 * torch.rand(D, generator=gen, device="cuda")).requires_grad_()
    x = (0.1 * torch.randn(B, D, L, generator=gen, device="cuda")).to(dtype).requires_grad_()
    go = torch.randn(B, D, L, generator=gen, device="cuda").to(dtype)

    def fused():
        y = fpscan_amd.pscan_softplus(z, rate, x)
        return torch.autograd.grad(y, (z, rate, x), go)

    def unfused():
        gates = torch.exp(-torch.nn.functional.softplus(z) * rate[None, :, None].to(dtype))
        y = fpscan_amd.pscan(gates, x)
        return torch.autograd.grad(y, (z, rate, x), go)

    res = {"workload": "c4fused: softplus-gate scan fwd+bwd B8 D1024 L65536",
           "dtype": SHORT[dtype]}
    for name, fn in (("fused", fused), ("unfused", unfused)):
        t = time_each(fn, WARM_CALLS, args.iters)
        p50 = percentile(t, 0.5)
        res[name] = {"p50_ms": round(p50, 5)}
    p50 = res["fused"]["p50_ms"]
    res["fused"]["gbps"] = round(8 * N * s / (p50 / 1e3) / 1e9, 1)
    res["fused"]["hbm_frac"] = round(8 * N * s / (p50 / 1e3) / 1e9 / HBM_PEAK_GBPS, 4)
    res["speedup_vs_unfused"] = round(res["unfused"]["p50_ms"] / p50, 3)
    print(json.dumps(res), flush=True)
    return res


def bench_dimwise(args):
    """dw: dimwise_forward (the reference module's contraction scan) at the headline shape,
    B8 D1024 L65536; 3 N s bytes per call (read Ax and Bx, write Bx; Bh, Wq, Wk are
    negligible). The reference's inputs (scans/contraction_scan.py:154-159). Beside it, the
    copy of the access pattern of the path the call takes: claimed 16 KiB tiles (tiled path,
    the default at this size) or eight-wave rows (row kernel)."""
    import fpscan_amd
    import fpscan_amd.ops as ops

    B, D, L = args.shape or (8, 1024, 65536)
    dtype = DTYPES[args.dtype or "bfloat16"]
    s = torch.empty((), dtype=dtype).element_size()
    N = B * D * L
    G = fpscan_amd.dimwise_groups(L)
    if G == 0:
        raise SystemExit(f"bench.py: dimwise_forward does not support seqlen {L}")
    gen = torch.Generator(device="cuda").manual_seed(2)
    ax = (0.99 + 0.01 * torch.rand(B, D, L, generator=gen, device="cuda")).to(dtype)
    bx0 = (torch.randn(B, D, L, generator=gen, device="cuda") / G).to(dtype)
    bh = (torch.randn(B, D, G, generator=gen, device="cuda") / G).to(dtype)
    wq = (0.01 * torch.rand(D, generator=gen, device="cuda")).to(dtype)
    wk = (0.01 * torch.rand(D, generator=gen, device="cuda")).to(dtype)
    bx = bx0.clone()
    # in place: Bx is restored from the same input before each timed call, outside the events.
    # Calls that rescan their own output instead time data that has grown to inf and NaN within
    # a few calls, which the tiled kernel ran up to 15 % faster than these inputs (a constant
    # bit pattern draws less power than random data).
    t = time_each(lambda: fpscan_amd.dimwise_forward(ax, bx, bh, wq, wk), WARM_CALLS, args.iters,
                  before=lambda: bx.copy_(bx0))
    p50 = percentile(t, 0.5)
    tiled = ops.dimwise_workspace_bytes(B, D, L, dtype) > 0
    entry = {"workload": f"dw: dimwise_forward B{B} D{D} L{L}", "dtype": SHORT[dtype],
             "path": "tiled" if tiled else "rows",
             "p50_ms": round(p50, 5), "gbps": round(3 * N * s / (p50 / 1e3) / 1e9, 1),
             "hbm_frac": round(3 * N * s / (p50 / 1e3) / 1e9 / HBM_PEAK_GBPS, 4)}
    # the copy of the path's access pattern (2 reads + 1 write of the same tensor size), timed
    # beside it
    import ctypes

    lib = ctypes.CDLL(os.path.join(os.path.dirname(fpscan_amd.__file__), "libfpscan_hip.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_probe_copy.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, i64, i64,
                                      vp, ctypes.c_size_t, vp]
    lib.fpscan_probe_copy.restype = ctypes.c_int
    lib.fpscan_probe_scratch_bytes.restype = ctypes.c_size_t
    del ax, bx0, bh, wq, wk, bx
    tensor_bytes = N * s
    # the probes copy whole 16 KiB tiles (rows of whole tiles for the row pattern), at most 4 GiB
    if (tensor_bytes % (16 << 10) or tensor_bytes > (1 << 32)
            or (not tiled and (L * s) % (16 << 10))):
        print(json.dumps(entry), flush=True)
        return entry
    src = torch.ones(2 * tensor_bytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty(tensor_bytes, dtype=torch.uint8, device="cuda")
    scratch = torch.zeros(lib.fpscan_probe_scratch_bytes(), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    pattern = PROBE_PATTERNS["tiles"] if tiled else PROBE_ROWS8

    def probe():
        st = lib.fpscan_probe_copy(pattern, 2, 1, src.data_ptr(), dst.data_ptr(), tensor_bytes,
                                   L * s, scratch.data_ptr(), scratch.numel(), stream)
        if st != 0:
            raise RuntimeError(f"fpscan_probe_copy status {st}")
    e = _timed_entry(probe, 3 * tensor_bytes, args.iters)
    entry["pattern_copy_tiles" if tiled else "pattern_copy_rows8"] = {
        k: e[k] for k in ("p50_ms", "gbps", "hbm_frac")}
    entry["of_pattern"] = round(entry["gbps"] / e["gbps"], 3)
    if tiled:
        # for comparison, the same copy in 8 KiB tiles with two 512-thread workgroups per CU
        # (a tile of one 2-byte chunk), which the tiled kernel does not use
        pattern = PROBE_TILES8
        e8 = _timed_entry(probe, 3 * tensor_bytes, args.iters)
        entry["pattern_copy_tiles8"] = {k: e8[k] for k in ("p50_ms", "gbps", "hbm_frac")}
    del src, dst, scratch
    print(json.dumps(entry), flush=True)
    return entry


PROBE_PATTERNS = {"tiles": 0, "blocks": 1, "rows": 2, "blocks_lookback": 3}  # fpscan_probe.h
PROBE_ROWS8 = 4  # eight-wave rows, 8 KiB rounds, two in flight: dimwise's row kernel
PROBE_TILES8 = 5  # 8 KiB tiles, 512-thread workgroups: a tile size the kernels do not use


def bench_ceiling(args):
    """ceiling: the access-pattern ceilings the scans are measured against. The library's
    bandwidth probes (include/fpscan_probe.h: copy kernels with the scans' access patterns and
    no scan) move 2 reads + 1 write (the forward's traffic) and 3 reads + 2 writes (the fused
    backward's) at the headline's per-tensor size (1 GiB: B8 D1024 L65536 bf16) and at the
    one-GPU share (128 MiB bf16, 256 MiB fp32), beside the forward and backward scans of the
    same sizes. p50 over --iters calls, GB/s of the bytes each moves."""
    import ctypes

    import fpscan_amd

    lib = ctypes.CDLL(os.path.join(os.path.dirname(fpscan_amd.__file__), "libfpscan_hip.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_probe_copy.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, i64, i64,
                                      vp, ctypes.c_size_t, vp]
    lib.fpscan_probe_copy.restype = ctypes.c_int
    lib.fpscan_probe_scratch_bytes.restype = ctypes.c_size_t
    lib.fpscan_probe_lookback_scratch_bytes.argtypes = [i64]
    lib.fpscan_probe_lookback_scratch_bytes.restype = ctypes.c_size_t
    import fpscan_amd.ops as ops
    cases = [("headline B8 D1024 L65536 bf16", 8, torch.bfloat16),
             ("share B1 D1024 L65536 bf16", 1, torch.bfloat16),
             ("share B1 D1024 L65536 f32", 1, torch.float32)]
    res = {"workload": "ceiling: access-pattern copy probes beside the scans", "iters": args.iters,
           "cases": []}
    for name, B, dtype in cases:
        D, L = 1024, 65536
        s = torch.empty((), dtype=dtype).element_size()
        tensor_bytes = B * D * L * s
        row_bytes = L * s
        entry = {"case": name, "tensor_bytes": tensor_bytes, "probes": {}}
        src = torch.ones(3 * tensor_bytes, dtype=torch.uint8, device="cuda")
        dst = torch.empty(2 * tensor_bytes, dtype=torch.uint8, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream
        for pname, pattern in PROBE_PATTERNS.items():
            scratch_bytes = (lib.fpscan_probe_lookback_scratch_bytes(tensor_bytes) if pname ==
                             "blocks_lookback" else lib.fpscan_probe_scratch_bytes())
            scratch = torch.zeros(scratch_bytes, dtype=torch.uint8, device="cuda")
            for nr, nw in ((2, 1), (3, 2)):
                def call():
                    st = lib.fpscan_probe_copy(pattern, nr, nw, src.data_ptr(), dst.data_ptr(),
                                               tensor_bytes, row_bytes, scratch.data_ptr(),
                                               scratch_bytes, stream)
                    if st != 0:
                        raise RuntimeError(f"fpscan_probe_copy status {st}")
                if pname == "blocks_lookback":
                    scratch.zero_()
                e = _timed_entry(call, (nr + nw) * tensor_bytes, args.iters)
                probe = {"p50_ms": e["p50_ms"], "gbps": e["gbps"], "hbm_frac": e["hbm_frac"]}
                if pname == "blocks_lookback":
                    polled, gave_up = scratch[:8].view(torch.int32).tolist()
                    calls = WARM_CALLS + args.iters
                    probe["tiles_polling_per_call"] = round(polled / calls, 1)
                    probe["tiles_per_call"] = tensor_bytes // (16 << 10)
                    probe["waits_given_up"] = gave_up
                entry["probes"][f"{pname}_{nr}r{nw}w"] = probe
            del scratch
        del src, dst
        gates, tokens, grad_out = make_inputs(B, D, L, dtype, "mamba", seed=5)
        out = torch.empty_like(tokens)
        y = fpscan_amd.scan_forward(gates, tokens)
        gg, gx = torch.empty_like(gates), torch.empty_like(gates)
        fwd = _timed_entry(lambda: fpscan_amd.scan_forward(gates, tokens, False, out),
                           3 * tensor_bytes, args.iters)
        bwd = _timed_entry(lambda: fpscan_amd.scan_backward(gates, y, grad_out, gg, gx),
                           5 * tensor_bytes, args.iters)
        entry["scan"] = {"fwd": {k: fwd[k] for k in ("p50_ms", "gbps", "hbm_frac")},
                         "bwd": {k: bwd[k] for k in ("p50_ms", "gbps", "hbm_frac")}}
        if B == 1:
            # the one-GPU share on each path forced: rows streamed (1) and tiles (2)
            for mode, label in ((1, "scan_streaming"), (2, "scan_tiled")):
                ops.set_tiling(mode)
                try:
                    f = _timed_entry(lambda: fpscan_amd.scan_forward(gates, tokens, False, out),
                                     3 * tensor_bytes, args.iters)
                    b = _timed_entry(lambda: fpscan_amd.scan_backward(gates, y, grad_out, gg, gx),
                                     5 * tensor_bytes, args.iters)
                finally:
                    ops.set_tiling(0)
                entry[label] = {"fwd": {k: f[k] for k in ("p50_ms", "gbps", "hbm_frac")},
                                "bwd": {k: b[k] for k in ("p50_ms", "gbps", "hbm_frac")}}
        del gates, tokens, grad_out, out, y, gg, gx
        print(json.dumps(entry), flush=True)
        res["cases"].append(entry)
    res["channel_last"] = _ceiling_channel_last(lib, args.iters)
    return res


def _ceiling_channel_last(lib, iters):
    """The channel-last tiled scan's pattern (fpscan_probe_copy_cl: chains of 64 columns, 16
    KiB tiles of one chain claimed per chain group) beside the channel-last scans, bf16
    (batch, 65536, 1024): batch 8 (128 chains, 1 GiB per tensor) and batch 1 (16 chains)."""
    import ctypes

    import fpscan_amd

    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_probe_copy_cl.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, i64, i64, i64,
                                         ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fpscan_probe_copy_cl.restype = ctypes.c_int
    out = []
    for B in (8, 1):
        L, D, dtype = 65536, 1024, torch.bfloat16
        s = 2
        tensor_bytes = B * L * D * s
        entry = {"case": f"channel-last ({B}, {L}, {D}) bf16", "chains": B * D // 64,
                 "tensor_bytes": tensor_bytes, "probes": {}}
        src = torch.ones(3 * tensor_bytes, dtype=torch.uint8, device="cuda")
        dst = torch.empty(2 * tensor_bytes, dtype=torch.uint8, device="cuda")
        scratch_bytes = lib.fpscan_probe_scratch_bytes()
        scratch = torch.zeros(scratch_bytes, dtype=torch.uint8, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream
        for nr, nw in ((2, 1), (3, 2)):
            def call():
                st = lib.fpscan_probe_copy_cl(nr, nw, src.data_ptr(), dst.data_ptr(), B, L, D * s,
                                              128, scratch.data_ptr(), scratch_bytes, stream)
                if st != 0:
                    raise RuntimeError(f"fpscan_probe_copy_cl status {st}")
            e = _timed_entry(call, (nr + nw) * tensor_bytes, iters)
            entry["probes"][f"cl_tiles_{nr}r{nw}w"] = {k: e[k] for k in ("p50_ms", "gbps",
                                                                          "hbm_frac")}
        del src, dst, scratch
        gen = torch.Generator(device="cuda").manual_seed(3)
        g = (0.99 + 0.01 * torch.rand(B, L, D, generator=gen, device="cuda")).to(dtype)
        x = (torch.randn(B, L, D, generator=gen, device="cuda") / L).to(dtype)
        go = torch.randn(B, L, D, generator=gen, device="cuda").to(dtype)
        y = fpscan_amd.scan_forward_channel_last(g, x)
        o = torch.empty_like(x)
        gg, gx = torch.empty_like(g), torch.empty_like(g)
        fwd = _timed_entry(lambda: fpscan_amd.scan_forward_channel_last(g, x, False, o),
                           3 * tensor_bytes, iters)
        bwd = _timed_entry(lambda: fpscan_amd.scan_backward_channel_last(g, y, go, gg, gx),
                           5 * tensor_bytes, iters)
        entry["scan"] = {"fwd": {k: fwd[k] for k in ("p50_ms", "gbps", "hbm_frac")},
                         "bwd": {k: bwd[k] for k in ("p50_ms", "gbps", "hbm_frac")}}
        del g, x, go, y, o, gg, gx
        print(json.dumps(entry), flush=True)
        out.append(entry)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c4", choices=["c1", "c2", "c3", "c4", "c5", "c4cl", "c5cl", "dw", "c4fused", "ceiling", "share", "rows"])
    ap.add_argument("--dtype", choices=list(DTYPES), default=None)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--flush", action="store_true",
                    help="c2: write 1 GiB before each timed call, so operands start uncached")
    ap.add_argument("--seqlens", type=int, nargs="+", default=None,
                    help="c2: the seqlens to sweep (default 32 .. 65536)")
    ap.add_argument("--batch", type=int, default=None,
                    help="c4cl/c5cl: override the batch (e.g. 1 for config 4's 8-GPU share)")
    ap.add_argument("--shape", default=None,
                    help="dw, rows: batch,dim,seqlen (dw defaults to the headline 8,1024,65536; "
                         "with --tiling 1 or 2 to time one path)")
    ap.add_argument("--no-fp32", action="store_true",
                    help="c4: skip the fp32 step reported beside the bf16 headline")
    ap.add_argument("--no-rows", action="store_true",
                    help="c4: skip the fused-gate, channel-last and dimwise figures reported "
                         "beside the headline")
    ap.add_argument("--no-configs", action="store_true",
                    help="c4: skip the B1 share and configs 2, 3 and 5 reported beside the "
                         "headline")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--launch", default=None, help="waves_per_row,ring_depth override")
    ap.add_argument("--tiling", type=int, choices=[0, 1, 2], default=0,
                    help="path selection: 0 automatic, 1 never tiled, 2 tiled where possible")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 5 device copies of a 1 GiB buffer: the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.shape is not None:
        try:
            args.shape = tuple(int(v) for v in args.shape.split(","))
        except ValueError:
            args.shape = ()
        if len(args.shape) != 3 or min(args.shape) < 1:
            ap.error("--shape takes three positive integers: batch,dim,seqlen")
    if args.workload == "rows" and args.shape is None:
        ap.error("--workload rows needs --shape batch,dim,seqlen")

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); rows are independent, so N GPUs would each run the "
              "same kernel on 1/N of the rows with no communication.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    if args.launch or args.tiling:
        import fpscan_amd.ops as ops

        if args.launch:
            w, u = (int(v) for v in args.launch.split(","))
            ops.set_launch_override(w, u)
        ops.set_tiling(args.tiling)

    if args.calibrate_copy:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    import fpscan_amd

    overruns_before = fpscan_amd.lookback_overruns()
    if args.workload == "c4":
        res = bench_headline(args)
    elif args.workload == "c2":
        res = bench_sweep(args)
    elif args.workload.endswith("cl"):
        res = bench_channel_last(args)
    elif args.workload == "dw":
        res = bench_dimwise(args)
    elif args.workload == "c4fused":
        res = bench_fused(args)
    elif args.workload == "ceiling":
        res = bench_ceiling(args)
    elif args.workload == "share":
        res = share_summary(args.steps)
    else:
        res = bench_shape(args)
    # health of the tiled kernels over the whole run: look-back waits that gave up (0 in a
    # correct run; each one leaves NaN outputs and about 10 ms of waiting in its call)
    overruns = fpscan_amd.lookback_overruns() - overruns_before
    if isinstance(res, dict):
        res["lookback_overruns"] = overruns
    if overruns:
        print(f"bench.py: {overruns} look-back waits gave up during the run", file=sys.stderr)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
