"""CPU checks of the narrowing fixtures that tests/test_rounding_gpu.py uses.

The GPU test compares every stored fp16/bf16 value with the exact result rounded to
nearest-even on the CPU. These checks show that the comparison can fail: on the same data,
the two plausible wrong rules -- truncation (round toward zero, e.g. a packing that drops the
low bits) and ties away from zero -- give different bits in many places, and the CPU rounding
itself is pinned on hand-worked values.
"""
import pytest
import torch

import oracle
from scan_helpers import (bits_equal, narrowed, rounding_counts, rounding_inputs, truncated)

HALF = [torch.bfloat16, torch.float16]


def ties_away(exact, dtype):
    """Round to nearest with ties away from zero (the planted wrong rule)."""
    t = torch.as_tensor(exact).double()
    lo = truncated(t, dtype)
    width = 2 if lo.element_size() == 2 else 4
    hi = (lo.view(torch.int16 if width == 2 else torch.int32) + 1).view(dtype)
    d_lo = (t - lo.double()).abs()
    d_hi = (hi.double() - t).abs()
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (d_lo > 0))
    return torch.where(pick_hi, hi, lo)


@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("L", [32, 1024, 65536])
@pytest.mark.parametrize("reverse", [False, True])
def test_fixtures_separate_nearest_even_from_other_rules(dtype, L, reverse):
    g, x = rounding_inputs((2, 3, L), dtype, reverse=reverse, seed=L)
    exact = oracle.scan_f64(g, x, reverse)
    inexact, ties = rounding_counts(exact, dtype)
    assert inexact >= exact.size // 5 and ties >= exact.size // 50
    want = narrowed(exact, dtype)
    assert not bits_equal(truncated(exact, dtype), want)
    assert not bits_equal(ties_away(exact, dtype), want)


def test_backward_fixture_products_stay_exact_and_need_rounding():
    """grad_gates = grad_tokens * out[t-1] must be exact in fp32 (below 2^24) and finite in
    fp16, yet not fit fp16/bf16."""
    for dtype in HALF:
        g, go = rounding_inputs((2, 3, 65536), dtype, reverse=True, step=3, seed=0)
        y = torch.randint(-7, 8, g.shape, generator=torch.Generator().manual_seed(1)).to(dtype)
        gg, gx = oracle.scan_bwd_f64(g, y, go)
        for v in (gg, gx):
            assert abs(v).max() < min(2 ** 24, 65504)
            assert rounding_counts(v, dtype)[0] > 0


def test_cpu_rounding_is_nearest_even_on_worked_values():
    # bf16 keeps 8 significant bits: 1 + 3 * 2^-9 lies between 1 and 1 + 2^-7, nearer the top
    # (truncation gives 1); 1 + 2^-8 is a tie between 1 (even) and 1 + 2^-7; 1 + 3 * 2^-8 a tie
    # between 1 + 2^-7 (odd) and 1 + 2^-6 (even)
    vals = [1 + 3 * 2 ** -9, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8)]
    want = [1 + 2 ** -7, 1.0, 1 + 2 ** -6, -1.0]
    assert narrowed(vals, torch.bfloat16).double().tolist() == want
    assert truncated(vals, torch.bfloat16).double().tolist() == [1.0, 1.0, 1 + 2 ** -7, -1.0]
    # fp16: integers from 2048 to 4096 are spaced 2, so odd ones are ties
    assert narrowed([2049.0, 2051.0, -2049.0, 3001.0], torch.float16).double().tolist() == \
        [2048.0, 2052.0, -2048.0, 3000.0]
    # fp16 subnormals are multiples of 2^-24: 3 * 2^-26 rounds up, 2^-25 is a tie to 0
    assert narrowed([3 * 2 ** -26, 2 ** -25], torch.float16).double().tolist() == [2 ** -24, 0.0]
