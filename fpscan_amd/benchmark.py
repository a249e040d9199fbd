"""Forward-scan latency sweep over sequence lengths: fpscan_amd against torch baselines.

    python -m fpscan_amd.benchmark [--batch 2] [--dim 256] [--dtype float32]
                                   [--seqlens 32 64 ... 65536] [--warmup 10] [--iters 100]
                                   [--compile-assoc] [--outdir DIR]

Same flags, table columns and plots as the reference's eval/benchmark.py:132-217: per seqlen
the p50 and p90 latency of every method (HIP events, one event pair per call), fpscan's
effective bandwidth 3 * batch * dim * seqlen * itemsize / p50, and the speedup of fpscan over
each baseline; then latency_vs_seqlen.png and speedup_vs_seqlen.png in --outdir (default: the
current directory). The table is a PrettyTable where that package is installed, plain aligned
text otherwise; plots need matplotlib and are skipped with a note without it. A baseline that
raises (for instance torch.associative_scan on a build that cannot run it eagerly) is
disabled for the remaining seqlens, as in the reference.
"""
from __future__ import annotations

import argparse
import math
import os
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

DEFAULT_SEQLENS = [32, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768, 65536]
DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def benchmark_fn(fn: Callable[[], object], warmup: int, iters: int) -> List[float]:
    """Per-call latency in ms: `warmup` untimed calls, then `iters` calls each bracketed by
    HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(iters)]
    for start, end in marks:
        start.record()
        fn()
        end.record()
    torch.cuda.synchronize()
    return [start.elapsed_time(end) for start, end in marks]


def percentiles(times: Optional[Sequence[float]]) -> Tuple[float, float]:
    """(p50, p90) with linear interpolation (torch.quantile's rule); NaNs without samples."""
    if not times:
        return math.nan, math.nan
    t = torch.tensor(list(times), dtype=torch.float64)
    return torch.quantile(t, 0.5).item(), torch.quantile(t, 0.9).item()


def make_inputs(batch: int, dim: int, seqlen: int, dtype: torch.dtype, device: str):
    """eval/benchmark.py's inputs: gates 0.99 + 0.01 U(0, 1), tokens N(0, 1) / seqlen."""
    gates = 0.99 + 0.01 * torch.rand(batch, dim, seqlen, device=device)
    tokens = torch.randn(batch, dim, seqlen, device=device) / seqlen
    return gates.to(dtype).contiguous(), tokens.to(dtype).contiguous()


def effective_bandwidth_gbps(batch: int, dim: int, seqlen: int, dtype: torch.dtype,
                             p50_ms: float) -> float:
    itemsize = torch.empty((), dtype=dtype).element_size()
    return 3 * batch * dim * seqlen * itemsize / 1e9 / (p50_ms / 1e3)


def build_methods(compile_assoc: bool) -> List[Tuple[str, Callable]]:
    import fpscan_amd
    from fpscan_amd.baselines import (ASSOCIATIVE_SCAN_AVAILABLE, parallel_scan_torch,
                                      torch_associative_scan)

    methods: List[Tuple[str, Callable]] = [
        ("fpscan", lambda g, x: fpscan_amd.scan_forward(g, x)),
        ("torch parallel", lambda g, x: parallel_scan_torch(g, x)),
    ]
    if ASSOCIATIVE_SCAN_AVAILABLE:
        assoc, label = torch_associative_scan, "torch.associative_scan"
        if compile_assoc:
            try:
                assoc = torch.compile(torch_associative_scan)
                label = "torch.associative_scan (compiled)"
            except Exception as exc:  # keep the eager baseline
                print(f"[warn] could not torch.compile associative_scan: {exc}")
        methods.append((label, lambda g, x, f=assoc: f(g, x)))
    else:
        print("[info] torch.associative_scan unavailable in this torch build; "
              "skipping that baseline.")
    return methods


def table_fields(method_names: Sequence[str]) -> List[str]:
    baselines = [n for n in method_names if n != "fpscan"]
    return (["seqlen"] + [f"{n} p50 (ms)" for n in method_names]
            + [f"{n} p90 (ms)" for n in method_names] + ["fpscan GB/s"]
            + [f"speedup vs {n}" for n in baselines])


def format_table(fields: Sequence[str], rows: Sequence[Sequence[float]]) -> str:
    """The result table: PrettyTable with 4 decimals where installed, the same cells as plain
    aligned text otherwise."""
    try:
        from prettytable import PrettyTable
    except ImportError:
        PrettyTable = None
    if PrettyTable is not None:
        table = PrettyTable()
        table.field_names = list(fields)
        table.float_format = "0.4"
        for row in rows:
            table.add_row(list(row))
        return str(table)

    def cell(v):
        return str(v) if isinstance(v, int) else f"{v:.4f}"

    cells = [list(fields)] + [[cell(v) for v in row] for row in rows]
    widths = [max(len(r[i]) for r in cells) for i in range(len(fields))]
    rule = "+" + "+".join("-" * (w + 2) for w in widths) + "+"
    lines = [rule]
    for k, r in enumerate(cells):
        lines.append("| " + " | ".join(c.rjust(w) for c, w in zip(r, widths)) + " |")
        if k == 0:
            lines.append(rule)
    lines.append(rule)
    return "\n".join(lines)


def _finite(xs, ys):
    return [(x, y) for x, y in zip(xs, ys) if y == y]


def plot_latency(seqlens, latencies: Dict[str, List[float]], names, path) -> bool:
    try:
        import matplotlib

        matplotlib.use("Agg")
        import matplotlib.pyplot as plt
    except ImportError:
        print(f"[info] matplotlib not installed; not writing {path}")
        return False
    fig = plt.figure(figsize=(8, 5))
    for name in names:
        pts = _finite(seqlens, latencies[name])
        if pts:
            plt.plot([p[0] for p in pts], [p[1] for p in pts], marker="o", label=name)
    plt.xscale("log", base=2)
    plt.yscale("log")
    plt.xlabel("sequence length")
    plt.ylabel("forward latency p50 (ms)")
    plt.title("Forward scan latency vs sequence length")
    plt.grid(True, which="both", alpha=0.3)
    plt.legend()
    plt.tight_layout()
    fig.savefig(path, dpi=120)
    plt.close(fig)
    print(f"wrote {path}")
    return True


def plot_speedup(seqlens, latencies: Dict[str, List[float]], baseline_names, path) -> bool:
    try:
        import matplotlib

        matplotlib.use("Agg")
        import matplotlib.pyplot as plt
    except ImportError:
        print(f"[info] matplotlib not installed; not writing {path}")
        return False
    fig = plt.figure(figsize=(8, 5))
    base = latencies["fpscan"]
    for name in baseline_names:
        pts = [(s, y / b) for s, b, y in zip(seqlens, base, latencies[name]) if b == b and y == y]
        if pts:
            plt.plot([p[0] for p in pts], [p[1] for p in pts], marker="o", label=f"vs {name}")
    plt.axhline(1.0, color="gray", linestyle="--", alpha=0.6)
    plt.xscale("log", base=2)
    plt.xlabel("sequence length")
    plt.ylabel("speedup (baseline / fpscan)")
    plt.title("fpscan forward speedup over baselines")
    plt.grid(True, which="both", alpha=0.3)
    plt.legend()
    plt.tight_layout()
    fig.savefig(path, dpi=120)
    plt.close(fig)
    print(f"wrote {path}")
    return True


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--batch", type=int, default=2)
    p.add_argument("--dim", type=int, default=256)
    p.add_argument("--dtype", choices=list(DTYPES), default="float32")
    p.add_argument("--seqlens", type=int, nargs="+", default=DEFAULT_SEQLENS)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--iters", type=int, default=100)
    p.add_argument("--compile-assoc", action="store_true",
                   help="torch.compile the associative_scan baseline")
    p.add_argument("--outdir", default=os.getcwd(), help="where the two plots go")
    return p.parse_args(argv)


def run(args: argparse.Namespace):
    """Runs the sweep; returns (table fields, rows, latencies per method)."""
    if not torch.cuda.is_available():
        raise SystemExit("This benchmark requires a HIP device.")
    dtype = DTYPES[args.dtype]
    methods = build_methods(args.compile_assoc)
    names = [n for n, _ in methods]
    baselines = [n for n in names if n != "fpscan"]
    print(f"device={torch.cuda.get_device_name()}  dtype={args.dtype}  batch={args.batch}  "
          f"dim={args.dim}  warmup={args.warmup}  iters={args.iters}")
    latencies: Dict[str, List[float]] = {n: [] for n in names}
    disabled: Dict[str, str] = {}
    rows = []
    for seqlen in args.seqlens:
        gates, tokens = make_inputs(args.batch, args.dim, seqlen, dtype, "cuda")
        p50s, p90s = {}, {}
        for name, fn in methods:
            times = None
            if name not in disabled:
                try:
                    times = benchmark_fn(lambda f=fn: f(gates, tokens), args.warmup, args.iters)
                except Exception as exc:
                    disabled[name] = str(exc)
                    print(f"    [disabled] {name}: {exc}")
            p50s[name], p90s[name] = percentiles(times)
            latencies[name].append(p50s[name])
        fp = p50s["fpscan"]
        gbps = (effective_bandwidth_gbps(args.batch, args.dim, seqlen, dtype, fp)
                if fp == fp else math.nan)
        speedups = [p50s[n] / fp if (p50s[n] == p50s[n] and fp == fp) else math.nan
                    for n in baselines]
        rows.append([seqlen] + [p50s[n] for n in names] + [p90s[n] for n in names] + [gbps]
                    + speedups)
        print(f"[{seqlen}] fpscan p50={fp:.4f}ms  "
              + "  ".join(f"{n}x{s:.2f}" for n, s in zip(baselines, speedups)), flush=True)
    return table_fields(names), rows, latencies


def main(argv=None) -> int:
    args = parse_args(argv)
    fields, rows, latencies = run(args)
    print(format_table(fields, rows))
    names = [f[: -len(" p50 (ms)")] for f in fields if f.endswith(" p50 (ms)")]
    os.makedirs(args.outdir, exist_ok=True)
    plot_latency(args.seqlens, latencies, names,
                 os.path.join(args.outdir, "latency_vs_seqlen.png"))
    plot_speedup(args.seqlens, latencies, [n for n in names if n != "fpscan"],
                 os.path.join(args.outdir, "speedup_vs_seqlen.png"))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
