"""The benchmark CLI (fpscan_amd.benchmark, the counterpart of the reference's
eval/benchmark.py) and its baselines (fpscan_amd.baselines, eval/baselines.py): the parts
that need no GPU run here; the sweep itself runs in the gpu-marked test at the end."""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from fpscan_amd import baselines, benchmark


@pytest.mark.parametrize("L", [1, 2, 31, 64, 100])
@pytest.mark.parametrize("reverse", [False, True])
def test_baselines_match_the_oracle(L, reverse):
    gen = torch.Generator().manual_seed(L)
    g = 0.5 + 0.5 * torch.rand(3, 4, L, generator=gen, dtype=torch.float64)
    x = torch.randn(3, 4, L, generator=gen, dtype=torch.float64)
    want = oracle.scan_f64(g, x, reverse)
    np.testing.assert_allclose(baselines.sequential_scan(g, x, reverse).numpy(), want,
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(baselines.parallel_scan_torch(g, x, reverse).numpy(), want,
                               rtol=1e-12, atol=1e-12)


def test_baselines_api_mirrors_the_reference():
    assert set(baselines.__all__) == {"sequential_scan", "parallel_scan_torch",
                                      "torch_associative_scan", "ASSOCIATIVE_SCAN_AVAILABLE",
                                      "BASELINES"}
    assert set(baselines.BASELINES) == {"sequential (oracle)", "torch parallel (hillis-steele)",
                                        "torch.associative_scan"}


def test_cli_defaults_are_the_references():
    a = benchmark.parse_args([])
    assert (a.batch, a.dim, a.dtype, a.warmup, a.iters, a.compile_assoc) == \
        (2, 256, "float32", 10, 100, False)
    assert a.seqlens == [2 ** k for k in range(5, 17)]
    b = benchmark.parse_args(["--seqlens", "64", "128", "--dtype", "bfloat16", "--outdir", "x"])
    assert b.seqlens == [64, 128] and b.dtype == "bfloat16" and b.outdir == "x"


def test_percentiles_interpolate_like_torch_quantile():
    assert benchmark.percentiles([1.0, 2.0, 3.0, 4.0]) == pytest.approx((2.5, 3.7))
    p50, p90 = benchmark.percentiles(None)
    assert math.isnan(p50) and math.isnan(p90)


def test_effective_bandwidth():
    # 3 * 2 * 256 * 1024 * 4 bytes in 0.001 s
    assert benchmark.effective_bandwidth_gbps(2, 256, 1024, torch.float32, 1.0) == \
        pytest.approx(3 * 2 * 256 * 1024 * 4 / 1e6)


def test_table_fields_and_plain_text_table():
    fields = benchmark.table_fields(["fpscan", "torch parallel"])
    assert fields == ["seqlen", "fpscan p50 (ms)", "torch parallel p50 (ms)", "fpscan p90 (ms)",
                      "torch parallel p90 (ms)", "fpscan GB/s", "speedup vs torch parallel"]
    text = benchmark.format_table(fields, [[32, 0.01, 0.5, 0.012, 0.6, 1.5, 50.0],
                                           [64, 0.011, math.nan, 0.013, math.nan, 2.5, math.nan]])
    lines = text.splitlines()
    assert all(f in lines[1] for f in fields)
    assert "0.0100" in text and "50.0000" in text and "nan" in text
    assert len({len(ln) for ln in lines}) == 1  # aligned


def test_plots_are_written(tmp_path):
    pytest.importorskip("matplotlib")
    seqlens = [32, 64, 128]
    lat = {"fpscan": [0.01, 0.011, math.nan], "torch parallel": [0.1, 0.2, 0.3]}
    a = os.path.join(tmp_path, "latency_vs_seqlen.png")
    b = os.path.join(tmp_path, "speedup_vs_seqlen.png")
    assert benchmark.plot_latency(seqlens, lat, list(lat), a)
    assert benchmark.plot_speedup(seqlens, lat, ["torch parallel"], b)
    for p in (a, b):
        with open(p, "rb") as f:
            assert f.read(8) == b"\x89PNG\r\n\x1a\n"


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)")
def test_cli_sweep_on_the_gpu(tmp_path, capsys):
    assert benchmark.main(["--seqlens", "32", "1024", "65536", "--iters", "5", "--warmup", "2",
                           "--outdir", str(tmp_path)]) == 0
    out = capsys.readouterr().out
    assert "fpscan p50 (ms)" in out and "seqlen 65536: fpscan" in out
    assert os.path.exists(os.path.join(tmp_path, "latency_vs_seqlen.png"))
    assert os.path.exists(os.path.join(tmp_path, "speedup_vs_seqlen.png"))
