"""Forward-scan latency sweep: fpscan_amd against the torch baselines, one row per seqlen.

    python -m fpscan_amd.benchmark [--batch 2] [--dim 256] [--dtype float32]
                                   [--seqlens 32 64 ... 65536] [--warmup 10] [--iters 100]
                                   [--compile-assoc] [--outdir DIR]

Interface kept from the reference's eval/benchmark.py, so its users find the same thing: the
flags and their defaults, the table's columns (p50 and p90 of each method, fpscan's GB/s at
3 * batch * dim * seqlen * itemsize bytes, the speedup of fpscan over each baseline) and the
two plots, latency_vs_seqlen.png and speedup_vs_seqlen.png, written to --outdir (here the
current directory by default).

How it runs: every seqlen gets fresh inputs with the reference's distributions; each method
is timed per call with a pair of HIP events around it on the current stream; a baseline that
raises once (for example torch.associative_scan where this torch build cannot run it
eagerly) is dropped for the rest of the sweep and its cells read nan. The table is a
PrettyTable when that package is installed and aligned plain text otherwise; the plots need
matplotlib and are skipped with a note without it.
"""
from __future__ import annotations

import argparse
import math
import os
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

DEFAULT_SEQLENS = [1 << k for k in range(5, 17)]
DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
FPSCAN = "fpscan"


def _say(msg: str) -> None:
    print(f"fpscan-bench: {msg}", flush=True)


# ------------------------------------------------------------------------- measurement
def benchmark_fn(fn: Callable[[], object], warmup: int, iters: int) -> List[float]:
    """Latency of each of `iters` calls in ms, after `warmup` untimed calls; one HIP event
    pair per call, recorded on the current stream (where the fpscan kernels run)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(2 * iters)]
    for i in range(iters):
        events[2 * i].record()
        fn()
        events[2 * i + 1].record()
    torch.cuda.synchronize()
    return [events[2 * i].elapsed_time(events[2 * i + 1]) for i in range(iters)]


def _quantile(sorted_xs: Sequence[float], q: float) -> float:
    pos = q * (len(sorted_xs) - 1)
    below = int(math.floor(pos))
    above = min(below + 1, len(sorted_xs) - 1)
    return sorted_xs[below] + (pos - below) * (sorted_xs[above] - sorted_xs[below])


def percentiles(times: Optional[Sequence[float]]) -> Tuple[float, float]:
    """(p50, p90), linearly interpolated between order statistics; nan, nan when a method
    produced no samples."""
    if not times:
        return math.nan, math.nan
    xs = sorted(float(t) for t in times)
    return _quantile(xs, 0.5), _quantile(xs, 0.9)


def make_inputs(batch: int, dim: int, seqlen: int, dtype: torch.dtype, device: str):
    """The reference benchmark's inputs: gates uniform in [0.99, 1), tokens N(0, 1) / seqlen,
    drawn in fp32, rounded to `dtype`, contiguous (batch, dim, seqlen)."""
    shape = (batch, dim, seqlen)
    gates = torch.rand(shape, device=device).mul_(0.01).add_(0.99)
    tokens = torch.randn(shape, device=device).div_(seqlen)
    return gates.to(dtype).contiguous(), tokens.to(dtype).contiguous()


def effective_bandwidth_gbps(batch: int, dim: int, seqlen: int, dtype: torch.dtype,
                             p50_ms: float) -> float:
    """GB/s of a forward scan: it reads gates and tokens and writes the output once."""
    moved = 3 * batch * dim * seqlen * torch.empty((), dtype=dtype).element_size()
    return moved / (p50_ms * 1e-3) / 1e9


# ------------------------------------------------------------------------- methods
@dataclass
class Method:
    name: str
    fn: Callable[[torch.Tensor, torch.Tensor], torch.Tensor]
    failure: Optional[str] = None  # set once the method raised; it is not run again


def build_methods(compile_assoc: bool) -> List[Method]:
    """fpscan first, then the baselines this torch build can run."""
    import fpscan_amd
    from fpscan_amd import baselines

    methods = [Method(FPSCAN, lambda g, x: fpscan_amd.scan_forward(g, x)),
               Method("torch parallel", baselines.parallel_scan_torch)]
    if not baselines.ASSOCIATIVE_SCAN_AVAILABLE:
        _say(f"torch {torch.__version__} has no associative_scan: that column is left out")
        return methods
    name, fn = "torch.associative_scan", baselines.torch_associative_scan
    if compile_assoc:
        try:
            fn = torch.compile(baselines.torch_associative_scan)
            name += " (compiled)"
        except Exception as exc:
            _say(f"torch.compile of associative_scan failed ({exc}); timing it eagerly")
    methods.append(Method(name, fn))
    return methods


# ------------------------------------------------------------------------- table
def table_fields(method_names: Sequence[str]) -> List[str]:
    others = [n for n in method_names if n != FPSCAN]
    return (["seqlen"]
            + [f"{n} p50 (ms)" for n in method_names]
            + [f"{n} p90 (ms)" for n in method_names]
            + ["fpscan GB/s"]
            + [f"speedup vs {n}" for n in others])


def _cell(v) -> str:
    return str(v) if isinstance(v, int) else f"{v:.4f}"


def format_table(fields: Sequence[str], rows: Sequence[Sequence[float]]) -> str:
    """PrettyTable (4 decimals) when installed; otherwise the same cells as aligned text
    between +---+ rules."""
    try:
        from prettytable import PrettyTable
    except ImportError:
        grid = [list(fields)] + [[_cell(v) for v in row] for row in rows]
        widths = [max(len(line[c]) for line in grid) for c in range(len(fields))]
        rule = "+".join([""] + ["-" * (w + 2) for w in widths] + [""])
        text = [rule]
        for n, line in enumerate(grid):
            text.append("|" + "|".join(f" {c:>{w}} " for c, w in zip(line, widths)) + "|")
            if n == 0:
                text.append(rule)
        return "\n".join(text + [rule])
    table = PrettyTable(list(fields))
    table.float_format = "0.4"
    for row in rows:
        table.add_row(list(row))
    return table.get_string()


# ------------------------------------------------------------------------- plots
def _pyplot():
    try:
        import matplotlib
    except ImportError:
        return None
    matplotlib.use("Agg")
    import matplotlib.pyplot as plt

    return plt


def _line_plot(path: str, series: Dict[str, List[Tuple[int, float]]], ylabel: str, title: str,
               log_y: bool, unity_line: bool) -> bool:
    plt = _pyplot()
    if plt is None:
        _say(f"no matplotlib here, {os.path.basename(path)} not written")
        return False
    fig, ax = plt.subplots(figsize=(7.5, 4.5))
    for label, points in series.items():
        if points:
            xs, ys = zip(*points)
            ax.plot(xs, ys, marker="s" if label == FPSCAN else "o", linewidth=1.5, label=label)
    if unity_line:
        ax.axhline(1.0, color="black", linewidth=0.8, linestyle=":")
    ax.set_xscale("log", base=2)
    if log_y:
        ax.set_yscale("log")
    ax.set_xlabel("seqlen")
    ax.set_ylabel(ylabel)
    ax.set_title(title)
    ax.grid(True, which="major", alpha=0.4)
    ax.legend(loc="best")
    fig.tight_layout()
    fig.savefig(path, dpi=150)
    plt.close(fig)
    _say(f"plot written to {path}")
    return True


def _finite(seqlens, values):
    return [(s, v) for s, v in zip(seqlens, values) if v == v]


def plot_latency(seqlens, latencies: Dict[str, List[float]], names, path) -> bool:
    """p50 latency of every method against seqlen, both axes logarithmic."""
    return _line_plot(path, {n: _finite(seqlens, latencies[n]) for n in names},
                      "p50 latency (ms)", "fpscan_amd forward scan: latency by seqlen",
                      log_y=True, unity_line=False)


def plot_speedup(seqlens, latencies: Dict[str, List[float]], baseline_names, path) -> bool:
    """Each baseline's p50 over fpscan's, against seqlen, with the break-even line at 1."""
    ours = latencies[FPSCAN]
    series = {f"vs {n}": _finite(seqlens, [b / f for f, b in zip(ours, latencies[n])])
              for n in baseline_names}
    return _line_plot(path, series, "speedup of fpscan (x)",
                      "fpscan_amd forward scan: speedup over baselines", log_y=False,
                      unity_line=True)


# ------------------------------------------------------------------------- sweep
@dataclass
class Sweep:
    names: List[str]
    rows: List[List[float]] = field(default_factory=list)
    latencies: Dict[str, List[float]] = field(default_factory=dict)


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--batch", type=int, default=2)
    p.add_argument("--dim", type=int, default=256)
    p.add_argument("--dtype", choices=list(DTYPES), default="float32")
    p.add_argument("--seqlens", type=int, nargs="+", default=DEFAULT_SEQLENS)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--iters", type=int, default=100)
    p.add_argument("--compile-assoc", action="store_true",
                   help="time torch.compile(torch_associative_scan) instead of the eager call")
    p.add_argument("--outdir", default=os.getcwd(), help="directory for the two PNG plots")
    return p.parse_args(argv)


def _time_method(m: Method, gates, tokens, args) -> Optional[List[float]]:
    if m.failure is not None:
        return None
    try:
        return benchmark_fn(lambda: m.fn(gates, tokens), args.warmup, args.iters)
    except Exception as exc:  # a baseline this build cannot run: drop it for the sweep
        m.failure = str(exc)
        _say(f"{m.name} raised and is dropped from the rest of the sweep: {exc}")
        return None


def run(args: argparse.Namespace):
    """Runs the sweep; returns (table fields, rows, per-method p50 latencies)."""
    if not torch.cuda.is_available():
        raise SystemExit("fpscan-bench: no HIP device visible")
    dtype = DTYPES[args.dtype]
    methods = build_methods(args.compile_assoc)
    sweep = Sweep([m.name for m in methods])
    sweep.latencies = {n: [] for n in sweep.names}
    _say(f"{torch.cuda.get_device_name()}, {args.dtype}, batch {args.batch}, dim {args.dim}, "
         f"{args.warmup} warmup + {args.iters} timed calls per method")
    for seqlen in args.seqlens:
        gates, tokens = make_inputs(args.batch, args.dim, seqlen, dtype, "cuda")
        stats = {m.name: percentiles(_time_method(m, gates, tokens, args)) for m in methods}
        ours = stats[FPSCAN][0]
        speedups = [stats[n][0] / ours for n in sweep.names if n != FPSCAN]
        gbps = effective_bandwidth_gbps(args.batch, args.dim, seqlen, dtype, ours)
        for n in sweep.names:
            sweep.latencies[n].append(stats[n][0])
        sweep.rows.append([seqlen] + [stats[n][0] for n in sweep.names]
                          + [stats[n][1] for n in sweep.names] + [gbps] + speedups)
        others = ", ".join(f"{s:.1f}x over {n}" for n, s in
                           zip([n for n in sweep.names if n != FPSCAN], speedups))
        _say(f"seqlen {seqlen}: fpscan {ours:.4f} ms ({gbps:.0f} GB/s); {others}")
        del gates, tokens
    return table_fields(sweep.names), sweep.rows, sweep.latencies


def main(argv=None) -> int:
    args = parse_args(argv)
    fields, rows, latencies = run(args)
    print(format_table(fields, rows), flush=True)
    names = list(latencies)
    os.makedirs(args.outdir, exist_ok=True)
    plot_latency(args.seqlens, latencies, names,
                 os.path.join(args.outdir, "latency_vs_seqlen.png"))
    plot_speedup(args.seqlens, latencies, [n for n in names if n != FPSCAN],
                 os.path.join(args.outdir, "speedup_vs_seqlen.png"))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
