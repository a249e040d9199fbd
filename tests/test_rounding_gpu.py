"""Bit-exact checks of the fp16/bf16 narrowing on every kernel family.

The reference narrows with __float2half / __float2bfloat16 (csrc/full_scan/conversion.h:7-13),
which round to nearest, ties to even. The normwise and elementwise bars of the other tests
cannot tell that rule from truncation (a truncating bf16 store is off by at most 2^-7
relative). Here every input makes each partial result an integer below 2^24 -- exact in fp32
in any combine order -- while most outputs need more significant bits than fp16/bf16 hold
and many sit exactly halfway between two neighbours (scan_helpers.rounding_inputs). So every
stored value must equal the exact result rounded once to nearest-even on the CPU, bit for
bit; each case also asserts that its data has inexact values and ties, so truncation or
ties-away-from-zero would fail it.

Paths: row scans streamed (short rows, 1..16 waves per row) and tiled (forced), forward,
reverse and the fused backward; channel-last one pass, segmented and tiled; the fused softplus
gate (rate 0 gives gates of exactly 1); dimwise_forward (unit gates and zero keys, where the
selection picks group 0 with weight 0).
"""
import numpy as np
import pytest
import torch

import fpscan_amd
import oracle
from fpscan_amd import ops
from scan_helpers import DEVICE, bits_equal, narrowed, rounding_counts, rounding_inputs

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]

HALF = [torch.bfloat16, torch.float16]


def assert_rounded(got, exact, dtype, what):
    inexact, ties = rounding_counts(exact, dtype)
    assert inexact > 0 and ties > 0, f"{what}: the data must need rounding (and hold ties)"
    want = narrowed(exact, dtype)
    got = got.cpu()
    if not bits_equal(got, want):
        bad = (got.view(torch.int16) != want.view(torch.int16)).nonzero()[:5].tolist()
        raise AssertionError(f"{what}: {len(bad)}+ values not rounded to nearest-even, first "
                             f"at {bad}: got {[got[tuple(i)].item() for i in bad]} want "
                             f"{[want[tuple(i)].item() for i in bad]}")


class tiling:
    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        ops.set_tiling(self.mode)

    def __exit__(self, *exc):
        ops.set_tiling(0)


def backward_inputs(shape, dtype, axis=-1, seed=0):
    """Saved output: small integers (their products with the integer grad_tokens stay exact in
    fp32 and below fp16's largest value); grad_out: rounding_inputs' tokens in the backward's
    processing order (it runs from the end)."""
    g, go = rounding_inputs(shape, dtype, axis=axis, reverse=True, step=3, seed=seed)
    gen = torch.Generator().manual_seed(seed + 1)
    out = torch.randint(-7, 8, shape, generator=gen).to(dtype)
    return g, out, go


# ------------------------------------------------------------------ row-major scans
@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("L", [32, 64, 128, 256, 512, 1024, 4096, 65536])
def test_row_scan_rounds_to_nearest_even(dtype, L):
    """Streaming kernels: short rows (L below 512), then 1, 2, 8 and 16 waves per row."""
    for rev in (False, True):
        g, x = rounding_inputs((2, 3, L), dtype, reverse=rev, seed=L)
        out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), reverse=rev)
        assert_rounded(out, oracle.scan_f64(g, x, rev), dtype, f"rows L{L} rev={rev}")


@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("L", [32, 256, 1024, 65536])
def test_row_backward_rounds_to_nearest_even(dtype, L):
    g, y, go = backward_inputs((2, 3, L), dtype, seed=L)
    gg, gx = fpscan_amd.scan_backward(g.to(DEVICE), y.to(DEVICE), go.to(DEVICE))
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, y, go)
    assert_rounded(gx, gx_ref, dtype, f"grad_tokens L{L}")
    assert_rounded(gg, gg_ref, dtype, f"grad_gates L{L}")


@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("shape", [(2, 3, 16384), (1, 2, 65536)], ids=str)
def test_tiled_row_scan_rounds_to_nearest_even(dtype, shape):
    with tiling(2):
        for rev in (False, True):
            g, x = rounding_inputs(shape, dtype, reverse=rev, seed=7)
            out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), reverse=rev)
            assert_rounded(out, oracle.scan_f64(g, x, rev), dtype, f"tiled {shape} rev={rev}")
        g, y, go = backward_inputs(shape, dtype, seed=8)
        gg, gx = fpscan_amd.scan_backward(g.to(DEVICE), y.to(DEVICE), go.to(DEVICE))
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, y, go)
    assert_rounded(gx, gx_ref, dtype, f"tiled grad_tokens {shape}")
    assert_rounded(gg, gg_ref, dtype, f"tiled grad_gates {shape}")


# ------------------------------------------------------------------ channel-last scans
CL_PATHS = {
    # (tiling mode, shape (batch, seqlen, dim) per itemsize) -> the path it takes
    "tiled": (2, {2: (2, 1000, 128), 4: (2, 1000, 128)}),
    "segmented": (1, {2: (2, 1000, 128), 4: (2, 1000, 128)}),
    "one-pass": (1, {2: (512, 40, 512), 4: (512, 40, 256)}),
}


@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("path", list(CL_PATHS))
def test_channel_last_rounds_to_nearest_even(dtype, path):
    mode, shapes = CL_PATHS[path]
    shape = shapes[torch.empty((), dtype=dtype).element_size()]
    with tiling(mode):
        for rev in (False, True):
            g, x = rounding_inputs(shape, dtype, axis=1, reverse=rev, seed=3)
            out = fpscan_amd.scan_forward_channel_last(g.to(DEVICE), x.to(DEVICE), reverse=rev)
            assert_rounded(out, oracle.scan_f64_channel_last(g, x, rev), dtype,
                           f"channel-last {path} rev={rev}")
        g, y, go = backward_inputs(shape, dtype, axis=1, seed=4)
        gg, gx = fpscan_amd.scan_backward_channel_last(g.to(DEVICE), y.to(DEVICE), go.to(DEVICE))
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, y, go)
    assert_rounded(gx, gx_ref, dtype, f"channel-last {path} grad_tokens")
    assert_rounded(gg, gg_ref, dtype, f"channel-last {path} grad_gates")


# ------------------------------------------------------------------ fused softplus gates
@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("L", [64, 1024, 65536])
def test_softplus_path_rounds_to_nearest_even(dtype, L):
    """rate 0: every gate is exp(-softplus(z) * 0) = 1 exactly, whatever z."""
    z = torch.randn(2, 3, L, generator=torch.Generator().manual_seed(L)).to(dtype)
    rate = torch.zeros(3)
    for rev in (False, True):
        g, x = rounding_inputs((2, 3, L), dtype, reverse=rev, seed=L + 1)
        out = fpscan_amd.scan_forward_softplus(z.to(DEVICE), rate.to(DEVICE), x.to(DEVICE),
                                               reverse=rev)
        assert_rounded(out, oracle.scan_f64(g, x, rev), dtype, f"softplus L{L} rev={rev}")
    g, y, go = backward_inputs((2, 3, L), dtype, seed=L + 2)
    gz, grate, gx = fpscan_amd.scan_backward_softplus(z.to(DEVICE), rate.to(DEVICE),
                                                      y.to(DEVICE), go.to(DEVICE))
    _, gx_ref = oracle.scan_bwd_f64(g, y, go)
    assert_rounded(gx, gx_ref, dtype, f"softplus grad_tokens L{L}")
    assert (gz.float() == 0).all(), "rate 0: d gate / d z is 0"


# ------------------------------------------------------------------ dimwise_forward
@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("L", [64, 512, 4096, 16384])
def test_dimwise_rounds_to_nearest_even(dtype, L):
    """Gates 1, Bh = Wq = Wk = 0: every score is 0, the first group wins with weight 0, so
    group g >= 1 adds group g-1's own total; group sums of integers up to +-200 (fp16: 500)
    need rounding in both types."""
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    step = 500 if dtype == torch.float16 else 200
    gen = torch.Generator().manual_seed(L)
    x = torch.randint(-step, step + 1, (2, 3, L), generator=gen).to(dtype)
    ones = torch.ones(2, 3, L, dtype=dtype)
    zeros_h = torch.zeros(2, 3, W * C, dtype=dtype)
    zeros_w = torch.zeros(3, dtype=dtype)
    exact = oracle.dimwise_f64(ones, x, zeros_h, zeros_w, zeros_w)
    bx = x.to(DEVICE)
    fpscan_amd.dimwise_forward(ones.to(DEVICE), bx, zeros_h.to(DEVICE), zeros_w.to(DEVICE),
                               zeros_w.to(DEVICE))
    assert np.abs(exact).max() < 2 ** 24 and np.all(exact == np.round(exact))
    assert_rounded(bx, exact, dtype, f"dimwise L{L}")
