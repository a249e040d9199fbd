"""GPU parity tests of the HIP scan against the CPU oracle (oracle/, pinned by
tests/test_oracle.py).

Mirrors the reference's tests/test_fpscan.py (forward at every seqlen, reverse, agreement with
the Hillis-Steele baseline, backward through autograd, the two validation errors) with its
tolerances (test_fpscan.py:18-22), and adds:

* the north-star bar, normwise max|y - y*| / max|y*| against the float64 oracle on the same
  rounded inputs: fp32 <= 1e-5, fp16 <= 5e-3, bf16 <= 2e-2 (outputs and both gradients);
* fp16/bf16 at every seqlen, reverse and backward in every dtype (unpinned in the reference);
* bit-exact known answers (tests/golden) and bit-exact size-independent properties at full
  size: reverse == flip(forward(flip)), scaling tokens by 2 scales outputs by exactly 2, the
  fused backward equals a reverse scan of the shifted gates;
* every benchmark configuration (bench.py's WORKLOADS, c1-c5) at its real shape, and the edge
  cases the reference does not test (ragged row counts, empty tensors, dim > 65535, `out=` and
  in-place use, first-gate NaN, side streams, every launch shape).
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

import fpscan_amd
import oracle
from fpscan_amd import ops

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]

from scan_helpers import (ALL_SEQLENS, DEVICE, DTYPES, NORM_TOL, REF_TOL, bits_equal, check,
                          make_inputs)

# ------------------------------------------------------------------ reference test suite
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", ALL_SEQLENS)
def test_forward_matches_oracle(dtype, seqlen):
    g, x = make_inputs(2, 4, seqlen, dtype, seed=seqlen)
    out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE))
    assert out.shape == x.shape and out.dtype == dtype and out.is_cuda
    check(out, oracle.scan_f64(g, x), dtype, f"fwd {dtype} L{seqlen}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", ALL_SEQLENS)
def test_reverse_matches_oracle(dtype, seqlen):
    g, x = make_inputs(2, 4, seqlen, dtype, seed=seqlen + 1)
    out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), reverse=True)
    check(out, oracle.scan_f64(g, x, reverse=True), dtype, f"rev {dtype} L{seqlen}")


@pytest.mark.parametrize("seqlen", [32, 256, 1024, 4096])
def test_agrees_with_torch_parallel_baseline(seqlen):
    g, x = make_inputs(2, 4, seqlen, torch.float32, seed=seqlen + 2)
    out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE))
    base = oracle.parallel_scan_torch(g.double(), x.double())
    torch.testing.assert_close(out.double().cpu(), base, **REF_TOL[torch.float32])


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", [32, 128, 512, 2048, 8192, 65536])
def test_backward_matches_oracle(dtype, seqlen):
    g, x = make_inputs(2, 4, seqlen, dtype, seed=seqlen + 3)
    w = torch.randn(g.shape, generator=torch.Generator().manual_seed(seqlen + 4))
    gd = g.to(DEVICE).requires_grad_()
    xd = x.to(DEVICE).requires_grad_()
    out = fpscan_amd.pscan(gd, xd)
    (out * w.to(DEVICE, dtype)).sum().backward()
    y_ref = oracle.scan_f64(g, x)
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, y_ref, w.to(dtype))
    check(xd.grad, gx_ref, dtype, f"grad_tokens {dtype} L{seqlen}")
    check(gd.grad, gg_ref, dtype, f"grad_gates {dtype} L{seqlen}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", [64, 4096])
def test_pscan_and_pscan_apply_agree_bit_for_bit(dtype, seqlen):
    """pscan runs the extension's C++ autograd function, PScan.apply the Python one; both
    launch the same kernels on the same saved tensors, so outputs and gradients are equal bit
    for bit, including when only one input requires a gradient."""
    g, x = make_inputs(3, 5, seqlen, dtype, seed=seqlen + 31)
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(3)).to(dtype).to(DEVICE)
    results = []
    for fn in (fpscan_amd.pscan, fpscan_amd.PScan.apply):
        gd = g.to(DEVICE).requires_grad_()
        xd = x.to(DEVICE).requires_grad_()
        y = fn(gd, xd)
        y.backward(go)
        results.append((y.detach(), gd.grad, xd.grad))
    for a, b in zip(*results):
        assert bits_equal(a, b)
    xd = x.to(DEVICE).requires_grad_()
    y = fpscan_amd.pscan(g.to(DEVICE), xd)  # gates without a gradient
    (gx,) = torch.autograd.grad(y, (xd,), go)
    assert bits_equal(gx, results[0][2])
    assert not fpscan_amd.pscan(g.to(DEVICE), x.to(DEVICE)).requires_grad


def test_non_power_of_two_seqlen_raises():
    g, x = make_inputs(1, 1, 32, torch.float32)
    with pytest.raises(RuntimeError):
        fpscan_amd.scan_forward(g[..., :30].contiguous().to(DEVICE),
                                x[..., :30].contiguous().to(DEVICE))


def test_non_contiguous_raises():
    g, x = make_inputs(2, 4, 64, torch.float32)
    with pytest.raises(RuntimeError):
        fpscan_amd.scan_forward(g.to(DEVICE).transpose(1, 2), x.to(DEVICE).transpose(1, 2))


# ------------------------------------------------------------------ known answers
def _golden(case, key):
    rows = [[float(Fraction(v)) for v in r] for r in case[key]]
    return torch.tensor(rows, dtype=torch.float64).unsqueeze(0)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_known_answers_bit_exact(known_answers, dtype):
    """Integer-valued cases (all-ones of scans/full_scan.py, segmented cumulative sums):
    exact in every dtype and every combine order, so the kernel must match bit for bit."""
    for case in known_answers:
        if case["name"].startswith("dyadic"):
            continue
        g = _golden(case, "gates").to(dtype)
        x = _golden(case, "tokens").to(dtype)
        for key, rev in (("forward", False), ("reverse", True)):
            out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), reverse=rev)
            want = torch.tensor(case[key], dtype=torch.float64).unsqueeze(0).to(dtype)
            assert bits_equal(out.cpu(), want), f"{case['name']} {key} {dtype}"


def test_known_answers_dyadic_fp32(known_answers):
    for case in known_answers:
        if not case["name"].startswith("dyadic"):
            continue
        g = _golden(case, "gates").float().to(DEVICE)
        x = _golden(case, "tokens").float().to(DEVICE)
        go = _golden(case, "grad_out").float().to(DEVICE)
        for key, rev in (("forward", False), ("reverse", True)):
            out = fpscan_amd.scan_forward(g, x, reverse=rev)
            want = np.array(case[key])[None]
            assert oracle.normwise_error(out, want) < 1e-6, f"{case['name']} {key}"
        y = fpscan_amd.scan_forward(g, x)
        gg, gx = fpscan_amd.scan_backward(g, y, go)
        assert oracle.normwise_error(gx, np.array(case["grad_tokens"])[None]) < 1e-6
        assert oracle.normwise_error(gg, np.array(case["grad_gates"])[None]) < 1e-6


# ------------------------------------------------------------------ agreement with the
# reference kernel's own arithmetic
@pytest.mark.parametrize("seqlen", [32, 64, 1024, 8192, 65536])
@pytest.mark.parametrize("reverse", [False, True])
def test_no_less_accurate_than_reference_kernel(seqlen, reverse):
    g, x = make_inputs(2, 8, seqlen, torch.float32, seed=seqlen + 11)
    out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), reverse=reverse)
    exact = oracle.scan_f64(g, x, reverse)
    ref_kernel = oracle.refkernel_f32(g, x, reverse)
    ours = oracle.normwise_error(out, exact)
    theirs = oracle.normwise_error(ref_kernel, exact)
    assert oracle.normwise_error(out, ref_kernel) < 1e-5
    assert ours <= 4 * theirs + 1e-7, f"ours {ours:.2e} vs reference kernel {theirs:.2e}"


# Relative size of one unit in the last place at the top of a binade, 2^-(p-1) for p
# significand bits: the largest normwise difference two correctly rounded results of nearly
# equal fp32 values can show.
ULP_REL = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _refkernel_scan(gates, tokens, reverse):
    """The reference kernel's arithmetic (fp32 accumulation in its combine order,
    full_scan.cu:77-176) rounded once to the tensors' dtype (conversion.h:7-13)."""
    return torch.from_numpy(oracle.refkernel_f32(gates, tokens, reverse)).to(gates.dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("seqlen", [32, 64, 1024, 8192, 65536])
@pytest.mark.parametrize("reverse", [False, True])
def test_half_types_agree_with_reference_kernel(dtype, seqlen, reverse):
    """fp16/bf16 forward and reverse against the reference kernel's own result: fp32
    accumulation, then one round-to-nearest-even to the input dtype. The two fp32 results
    differ only in combine order, so after rounding they agree bit for bit almost everywhere
    and by one unit in the last place elsewhere; and ours is no less accurate against the
    float64 recurrence."""
    g, x = make_inputs(2, 8, seqlen, dtype, seed=seqlen + 11)
    out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), reverse=reverse).cpu()
    ref_kernel = _refkernel_scan(g, x, reverse)
    exact = oracle.scan_f64(g, x, reverse)
    same = (out.view(torch.int16) == ref_kernel.view(torch.int16)).double().mean().item()
    assert same >= 0.995, f"only {same:.4%} of the outputs equal the reference kernel's bits"
    assert oracle.normwise_error(out, ref_kernel) <= ULP_REL[dtype]
    ours = oracle.normwise_error(out, exact)
    theirs = oracle.normwise_error(ref_kernel, exact)
    assert ours <= 1.25 * theirs + 1e-7, f"ours {ours:.2e} vs reference kernel {theirs:.2e}"


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", [32, 1024, 8192, 65536])
def test_backward_agrees_with_reference_composition(dtype, seqlen):
    """The fused backward against the reference's own backward on the same saved output:
    PScan.backward's composition (fpscan/ops.py:69-83) -- shifted gates, the reference kernel's
    reverse scan rounded to the dtype, then grad_gates = out[t-1] * grad_tokens in the dtype's
    arithmetic (grad_tokens rounded before the product). The fused kernel keeps grad_tokens in
    fp32 for the product, so grad_gates may differ by one more rounding; both gradients must
    stay within that and be no less accurate against the float64 adjoint."""
    g, x = make_inputs(2, 8, seqlen, dtype, seed=seqlen + 21)
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(seqlen)).to(dtype)
    y = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE))
    gg, gx = fpscan_amd.scan_backward(g.to(DEVICE), y, go.to(DEVICE))
    gg, gx, y = gg.cpu(), gx.cpu(), y.cpu()
    gg_ref, gx_ref = oracle.pscan_backward_composed(g, y, go, _refkernel_scan)
    gg64, gx64 = oracle.scan_bwd_f64(g, y, go)
    tol = max(ULP_REL[dtype], 1e-5)
    assert oracle.normwise_error(gx, gx_ref) <= tol, "grad_tokens vs the reference composition"
    assert oracle.normwise_error(gg, gg_ref) <= 2 * tol, "grad_gates vs the reference composition"
    for name, ours, theirs in (("grad_tokens", gx, gx_ref), ("grad_gates", gg, gg_ref)):
        want = gx64 if name == "grad_tokens" else gg64
        e_ours, e_ref = oracle.normwise_error(ours, want), oracle.normwise_error(theirs, want)
        bound = (4 * e_ref + 1e-7) if dtype == torch.float32 else (1.25 * e_ref + 1e-7)
        assert e_ours <= bound, f"{name}: ours {e_ours:.2e} vs reference composition {e_ref:.2e}"


# ------------------------------------------------------------------ edge cases
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", [32, 64, 128, 256, 512, 4096, 65536])
def test_ragged_row_counts(dtype, seqlen):
    """3 x 5 = 15 rows: not a multiple of the rows per block or per wave."""
    g, x = make_inputs(3, 5, seqlen, dtype, seed=7 * seqlen)
    out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE))
    check(out, oracle.scan_f64(g, x), dtype, "ragged")
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(5)).to(dtype)
    gg, gx = fpscan_amd.scan_backward(g.to(DEVICE), out, go.to(DEVICE))
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, out.cpu(), go)
    check(gx, gx_ref, dtype, "ragged grad_tokens")
    check(gg, gg_ref, dtype, "ragged grad_gates")


@pytest.mark.parametrize("shape", [(0, 4, 64), (2, 0, 64), (0, 0, 32)])
def test_empty_tensors(shape):
    g = torch.rand(shape, device=DEVICE)
    out = fpscan_amd.scan_forward(g, g.clone())
    assert out.shape == shape
    gg, gx = fpscan_amd.scan_backward(g, g.clone(), g.clone())
    assert gg.shape == gx.shape == shape


@pytest.mark.parametrize("seqlen", [32, 512])
def test_dim_beyond_grid_y_limit(seqlen):
    """dim > 65535 failed in the reference (gridDim.y); rows here are a 1-d range."""
    g, x = make_inputs(1, 70000, seqlen, torch.float32, seed=3)
    out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE))
    check(out, oracle.scan_f64(g, x), torch.float32, "dim 70000")


def test_out_parameter_is_written_and_returned():
    g, x = make_inputs(2, 4, 1024, torch.float32, seed=9)
    out = torch.full((2, 4, 1024), float("nan"), device=DEVICE)
    ret = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), out=out)
    assert ret is out
    check(out, oracle.scan_f64(g, x), torch.float32, "out=")


def test_in_place_on_tokens():
    g, x = make_inputs(2, 4, 4096, torch.bfloat16, seed=10)
    xd = x.to(DEVICE)
    fpscan_amd.scan_forward(g.to(DEVICE), xd, out=xd)
    check(xd, oracle.scan_f64(g, x), torch.bfloat16, "in place")


@pytest.mark.parametrize("bad", ["dtype_mix", "shape_mix", "out_dtype", "out_shape", "dim2",
                                 "cpu_mix", "int_dtype", "out_noncontig"])
def test_validation_errors(bad):
    g, x = make_inputs(2, 4, 64, torch.float32)
    g, x = g.to(DEVICE), x.to(DEVICE)
    out = None
    if bad == "dtype_mix":
        g = g.half()
    elif bad == "shape_mix":
        g = g[:1].contiguous()
    elif bad == "out_dtype":
        out = torch.empty_like(x, dtype=torch.float16)
    elif bad == "out_shape":
        out = torch.empty(2, 4, 32, device=DEVICE)
    elif bad == "dim2":
        g, x = g[0], x[0]
    elif bad == "cpu_mix":
        g = g.cpu()
    elif bad == "int_dtype":
        g, x = g.int(), x.int()
    elif bad == "out_noncontig":
        out = torch.empty(2, 64, 4, device=DEVICE).transpose(1, 2)
    with pytest.raises(RuntimeError):
        fpscan_amd.scan_forward(g, x, out=out)


def test_backward_rejects_aliased_outputs():
    g, x = make_inputs(1, 4, 64, torch.float32)
    g, x = g.to(DEVICE), x.to(DEVICE)
    y = fpscan_amd.scan_forward(g, x)
    go = torch.randn_like(y)
    with pytest.raises(RuntimeError):
        fpscan_amd.scan_backward(g, y, go, grad_gates=go)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", [64, 4096, 65536])
def test_first_processed_gate_is_ignored(dtype, seqlen):
    """full_scan.cu:96: the first element's gate (gates[0] forward, gates[L-1] reverse) is
    replaced by 1, so even NaN there leaves the result finite and unchanged."""
    g, x = make_inputs(2, 4, seqlen, dtype, seed=seqlen)
    base_f = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE))
    base_r = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE), reverse=True)
    gf, gr = g.clone(), g.clone()
    gf[..., 0] = float("nan")
    gr[..., -1] = float("nan")
    assert bits_equal(fpscan_amd.scan_forward(gf.to(DEVICE), x.to(DEVICE)), base_f)
    assert bits_equal(fpscan_amd.scan_forward(gr.to(DEVICE), x.to(DEVICE), reverse=True), base_r)


def test_runs_on_the_current_stream():
    g, x = make_inputs(4, 64, 8192, torch.float32, seed=12)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        out = fpscan_amd.scan_forward(gd, xd)
        ev = torch.cuda.Event()
        ev.record(side)
    ev.synchronize()
    check(out, oracle.scan_f64(g, x), torch.float32, "side stream")


@pytest.mark.parametrize("waves,ring", [(w, u) for w in (1, 2, 4, 8, 16) for u in (1, 2, 3, 4)])
def test_every_launch_shape(waves, ring):
    """All (waves per row, ring depth) variants: exact on integer data, oracle-close on random
    data, forward, reverse and backward, every dtype."""
    try:
        ops.set_launch_override(waves, ring)
        for dtype in DTYPES:
            L = 32768 if dtype == torch.float32 else 65536  # >= 16 sub-chunks per row
            gen = torch.Generator().manual_seed(waves * 10 + ring)
            gi = (torch.randint(0, 16, (1, 3, L), generator=gen) > 0).to(dtype)
            xi = torch.randint(-3, 4, (1, 3, L), generator=gen).to(dtype)
            for rev in (False, True):
                out = fpscan_amd.scan_forward(gi.to(DEVICE), xi.to(DEVICE), reverse=rev)
                want = torch.from_numpy(oracle.scan_f64(gi, xi, rev))
                if dtype == torch.float32 or want.abs().max() < 256:
                    assert bits_equal(out.cpu(), want.to(dtype)), (dtype, rev)
            g, x = make_inputs(1, 3, L, dtype, seed=waves + ring)
            out = fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE))
            check(out, oracle.scan_f64(g, x), dtype, f"W{waves} U{ring} fwd")
            go = torch.randn(g.shape, generator=gen).to(dtype)
            gg, gx = fpscan_amd.scan_backward(g.to(DEVICE), out, go.to(DEVICE))
            gg_ref, gx_ref = oracle.scan_bwd_f64(g, out.cpu(), go)
            check(gx, gx_ref, dtype, f"W{waves} U{ring} grad_tokens")
            check(gg, gg_ref, dtype, f"W{waves} U{ring} grad_gates")
    finally:
        ops.set_launch_override(0, 0)


# ------------------------------------------------------------------ size-independent,
# bit-exact properties
def _properties(g, x, go, rows_checked=0):
    """Checks at any size: (1) reverse == flip(forward(flip)); (2) tokens*2 -> out*2 exactly;
    (3) grad_tokens == reverse scan of the shifted gates, bit for bit, and for fp32
    grad_gates == out[t-1] * grad_tokens bit for bit."""
    dtype = g.dtype
    out = fpscan_amd.scan_forward(g, x)
    rev = fpscan_amd.scan_forward(g, x, reverse=True)
    assert bits_equal(rev, fpscan_amd.scan_forward(g.flip(-1), x.flip(-1)).flip(-1))
    # doubling commutes with rounding except for fp16 subnormal results (fixed spacing below
    # 2^-14; bf16 and fp32 share fp32's exponent range): fp16 compares normal elements only
    y2 = fpscan_amd.scan_forward(g, x * 2)
    if dtype == torch.float16:
        normal = out.abs() >= 2.0 ** -13
        assert normal.float().mean() > 0.5
        assert bits_equal(y2[normal], (out * 2)[normal])
    else:
        assert bits_equal(y2, out * 2)
    gg, gx = fpscan_amd.scan_backward(g, out, go)
    shifted = torch.cat([g[..., 1:], torch.ones_like(g[..., :1])], dim=-1)
    assert bits_equal(gx, fpscan_amd.scan_forward(shifted, go, reverse=True))
    if dtype == torch.float32:
        prev = torch.cat([torch.zeros_like(out[..., :1]), out[..., :-1]], dim=-1)
        assert bits_equal(gg, prev * gx)
    if rows_checked:
        rows = g.shape[0] * g.shape[1]
        idx = torch.linspace(0, rows - 1, rows_checked).long()
        L = g.shape[-1]
        gs = g.reshape(rows, L)[idx].cpu()
        xs = x.reshape(rows, L)[idx].cpu()
        gos = go.reshape(rows, L)[idx].cpu()
        y_ref = oracle.scan_f64(gs, xs)
        check(out.reshape(rows, L)[idx], y_ref, dtype, "subset out")
        check(rev.reshape(rows, L)[idx], oracle.scan_f64(gs, xs, True), dtype, "subset rev")
        gg_ref, gx_ref = oracle.scan_bwd_f64(gs, y_ref, gos)
        check(gx.reshape(rows, L)[idx], gx_ref, dtype, "subset grad_tokens")
        check(gg.reshape(rows, L)[idx], gg_ref, dtype, "subset grad_gates")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_properties_mid_size(dtype):
    g, x = make_inputs(2, 64, 16384, dtype, seed=21)
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(22)).to(dtype)
    _properties(g.to(DEVICE), x.to(DEVICE), go.to(DEVICE), rows_checked=16)


# ------------------------------------------------------------------ benchmark configs
def test_config1_b2_d256_l1024_fp32():
    g, x = make_inputs(2, 256, 1024, torch.float32, seed=0)
    check(fpscan_amd.scan_forward(g.to(DEVICE), x.to(DEVICE)), oracle.scan_f64(g, x),
          torch.float32, "config 1")


@pytest.mark.parametrize("seqlen", ALL_SEQLENS)
def test_config2_sweep_b2_d256_fp32(seqlen):
    g, x = make_inputs(2, 256, seqlen, torch.float32, seed=seqlen)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    check(fpscan_amd.scan_forward(gd, xd), oracle.scan_f64(g, x), torch.float32, "c2 fwd")
    check(fpscan_amd.scan_forward(gd, xd, reverse=True), oracle.scan_f64(g, x, True),
          torch.float32, "c2 rev")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_config3_b4_d512_l8192_fwd_bwd(dtype):
    g, x = make_inputs(4, 512, 8192, dtype, seed=3)
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(33)).to(dtype)
    gd = g.to(DEVICE).requires_grad_()
    xd = x.to(DEVICE).requires_grad_()
    out = fpscan_amd.pscan(gd, xd)
    gg, gx = torch.autograd.grad(out, (gd, xd), go.to(DEVICE))
    y_ref = oracle.scan_f64(g, x)
    check(out, y_ref, dtype, "c3 out")
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, y_ref, go)
    check(gx, gx_ref, dtype, "c3 grad_tokens")
    check(gg, gg_ref, dtype, "c3 grad_gates")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_mid_size_rows_of_64_sub_chunks_fwd_rev_bwd(dtype):
    """16-64 MiB tensors whose rows hold 64 sub-chunks (4 rounds of a 16-wave row) stream as
    8-wave rows by default, forward, reverse and backward: checked against the oracle."""
    B, D, L = (2, 256, 16384) if dtype == torch.float32 else (2, 128, 32768)
    g, x = make_inputs(B, D, L, dtype, seed=L + 5)
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(55)).to(dtype)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    y = fpscan_amd.scan_forward(gd, xd)
    y_ref = oracle.scan_f64(g, x)
    check(y, y_ref, dtype, "mid fwd")
    check(fpscan_amd.scan_forward(gd, xd, reverse=True), oracle.scan_f64(g, x, True), dtype,
          "mid rev")
    gg, gx = torch.empty_like(gd), torch.empty_like(gd)
    fpscan_amd.scan_backward(gd, y, go.to(DEVICE), gg, gx)
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, y.cpu().double(), go)
    check(gx, gx_ref, dtype, "mid grad_tokens")
    check(gg, gg_ref, dtype, "mid grad_gates")


def _bench_inputs(batch, dim, seqlen, dtype, dist, seed):
    import bench

    return bench.make_inputs(batch, dim, seqlen, dtype, dist, seed=seed, device=DEVICE)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_config4_headline_b8_d1024_l65536(dtype):
    g, x, go = _bench_inputs(8, 1024, 65536, dtype, "mamba", seed=4)
    _properties(g, x, go, rows_checked=48)


def test_config5_b64_d4096_l256_and_transposed_layout():
    g, x, go = _bench_inputs(64, 4096, 256, torch.float32, "sigmoid", seed=5)
    out = fpscan_amd.scan_forward(g, x)
    check(out, oracle.scan_f64(g, x), torch.float32, "c5")
    # (batch, seqlen, dim) data: transpose in and out around the call (README.md:94-99)
    gt, xt = g.mT.contiguous(), x.mT.contiguous()
    out_t = fpscan_amd.scan_forward(gt.mT.contiguous(), xt.mT.contiguous()).mT.contiguous()
    assert bits_equal(out_t, out.mT.contiguous())
    gg, gx = fpscan_amd.scan_backward(g, out, go)
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, out, go)
    check(gx, gx_ref, torch.float32, "c5 grad_tokens")
    check(gg, gg_ref, torch.float32, "c5 grad_gates")


# ------------------------------------------------------------------ rows of one sub-chunk
# From 32768 such rows (65536 in the backward) each row gets a 64-thread block of its own; a
# launch override sends the same call to the 4-rows-per-block launch, which computes each row
# the same way.
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_one_row_per_block_matches_oracle_and_four_rows_per_block(dtype):
    L = 256 if dtype == torch.float32 else 512  # one sub-chunk
    B, D = 2, 32768 + 21  # ragged: not a multiple of 4 rows
    g, x = make_inputs(B, D, L, dtype, seed=L + 1)
    g[0, 100, 0] = float("nan")  # the forward's first gate of a row: never used there
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(8)).to(dtype)
    gd, xd, god = g.to(DEVICE), x.to(DEVICE), go.to(DEVICE)
    y = fpscan_amd.scan_forward(gd, xd)
    yr = fpscan_amd.scan_forward(gd, xd, reverse=True)
    gg, gx = fpscan_amd.scan_backward(gd, y, god)
    try:
        ops.set_launch_override(1, 1)
        y4 = fpscan_amd.scan_forward(gd, xd)
        yr4 = fpscan_amd.scan_forward(gd, xd, reverse=True)
        gg4, gx4 = fpscan_amd.scan_backward(gd, y, god)
    finally:
        ops.set_launch_override(0, 0)
    for got, want, what in ((y, y4, "fwd"), (yr, yr4, "rev"), (gg, gg4, "grad_gates"),
                            (gx, gx4, "grad_tokens")):
        assert bits_equal(got, want), f"{what}: one row per block differs from four"
    assert torch.isfinite(y).all() and torch.isfinite(gx).all()
    rows = torch.cat([torch.arange(0, 8), torch.arange(D - 8, D + 8),
                      torch.arange(2 * D - 8, 2 * D)])
    g2, x2, go2 = (t.reshape(B * D, L)[rows] for t in (g, x, go))
    check(y.reshape(B * D, L)[rows], oracle.scan_f64(g2, x2), dtype, "one-row blocks fwd")
    check(yr.reshape(B * D, L)[rows], oracle.scan_f64(g2, x2, True), dtype, "one-row blocks rev")
    gg_ref, gx_ref = oracle.scan_bwd_f64(g2, y.reshape(B * D, L)[rows].cpu(), go2)
    check(gx.reshape(B * D, L)[rows], gx_ref, dtype, "one-row blocks grad_tokens")
    check(gg.reshape(B * D, L)[rows], gg_ref, dtype, "one-row blocks grad_gates")


@pytest.mark.parametrize("dtype,L", [(torch.float32, 16384), (torch.bfloat16, 8192)], ids=str)
def test_eight_wave_rows_with_padded_strides_through_the_c_abi(dtype, L):
    """16-64 MiB tensors of rows with 16-64 sub-chunks (8 waves per row by default) in a
    larger buffer: forward and backward against the oracle on sampled rows, padding
    untouched."""
    lib = _abi()
    B, D = 2, 1024 if dtype == torch.bfloat16 else 256
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    sd = L + 8 * vec
    sb = D * sd + 4 * vec
    g, x = make_inputs(B, D, L, dtype, seed=L + 13)
    go = torch.randn(B, D, L, generator=torch.Generator().manual_seed(14)).to(dtype)

    def embed(t, fill):
        buf = torch.full((B * sb,), fill, dtype=dtype)
        buf.as_strided((B, D, L), (sb, sd, 1)).copy_(t)
        return buf.to(DEVICE)

    def view(buf):
        return buf.cpu().as_strided((B, D, L), (sb, sd, 1))

    gb, xb, gob = embed(g, 7.0), embed(x, 7.0), embed(go, 7.0)
    outb, ggb, gxb = (embed(torch.zeros_like(x), -3.0) for _ in range(3))
    stream = torch.cuda.current_stream().cuda_stream
    code = _CODE[dtype]
    assert lib.fpscan_scan_fwd(gb.data_ptr(), xb.data_ptr(), outb.data_ptr(), B, D, L, sb, sd,
                               code, 0, None, 0, stream) == 0
    assert lib.fpscan_scan_bwd(gb.data_ptr(), outb.data_ptr(), gob.data_ptr(), ggb.data_ptr(),
                               gxb.data_ptr(), B, D, L, sb, sd, code, None, 0, stream) == 0
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, D - 1, D, 2 * D - 1])
    out = view(outb).reshape(B * D, L)[rows]
    g2, x2, go2 = (t.reshape(B * D, L)[rows] for t in (g, x, go))
    check(out, oracle.scan_f64(g2, x2), dtype, "strided 8-wave fwd")
    gg_ref, gx_ref = oracle.scan_bwd_f64(g2, out, go2)
    check(view(gxb).reshape(B * D, L)[rows], gx_ref, dtype, "strided 8-wave grad_tokens")
    check(view(ggb).reshape(B * D, L)[rows], gg_ref, dtype, "strided 8-wave grad_gates")
    mask = torch.ones(B * sb, dtype=torch.bool)
    mask.as_strided((B, D, L), (sb, sd, 1)).fill_(False)
    for buf, what in ((outb, "out"), (ggb, "grad_gates"), (gxb, "grad_tokens")):
        assert (buf.cpu()[mask] == -3.0).all(), f"padding of {what} was written"


def test_one_row_per_block_with_padded_strides_through_the_c_abi():
    """Rows of one sub-chunk in a larger buffer (stride_d = L + pad, stride_b = dim * stride_d
    + pad2): each 64-thread block finds its row through the strides, forward and backward,
    and the padding comes back untouched."""
    lib = _abi()
    B, D, L = 2, 32768 + 5, 256
    sd, sb = L + 32, (32768 + 5) * (L + 32) + 16
    g, x = make_inputs(B, D, L, torch.float32, seed=77)
    go = torch.randn(B, D, L, generator=torch.Generator().manual_seed(78))

    def embed(t, fill):
        buf = torch.full((B * sb,), fill, dtype=torch.float32)
        buf.as_strided((B, D, L), (sb, sd, 1)).copy_(t)
        return buf.to(DEVICE)

    def view(buf):
        return buf.cpu().as_strided((B, D, L), (sb, sd, 1))

    gb, xb, gob = embed(g, 7.0), embed(x, 7.0), embed(go, 7.0)
    outb, ggb, gxb = (embed(torch.zeros_like(x), -3.0) for _ in range(3))
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.fpscan_scan_fwd(gb.data_ptr(), xb.data_ptr(), outb.data_ptr(), B, D, L, sb, sd,
                               0, 0, None, 0, stream) == 0
    assert lib.fpscan_scan_bwd(gb.data_ptr(), outb.data_ptr(), gob.data_ptr(), ggb.data_ptr(),
                               gxb.data_ptr(), B, D, L, sb, sd, 0, None, 0, stream) == 0
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(0, 4), torch.arange(D - 4, D + 4), torch.arange(2 * D - 4, 2 * D)])
    out = view(outb).reshape(B * D, L)[rows]
    g2, x2, go2 = (t.reshape(B * D, L)[rows] for t in (g, x, go))
    check(out, oracle.scan_f64(g2, x2), torch.float32, "strided one-row blocks fwd")
    gg_ref, gx_ref = oracle.scan_bwd_f64(g2, out, go2)
    check(view(gxb).reshape(B * D, L)[rows], gx_ref, torch.float32, "strided grad_tokens")
    check(view(ggb).reshape(B * D, L)[rows], gg_ref, torch.float32, "strided grad_gates")
    mask = torch.ones(B * sb, dtype=torch.bool)
    mask.as_strided((B, D, L), (sb, sd, 1)).fill_(False)
    for buf, what in ((outb, "out"), (ggb, "grad_gates"), (gxb, "grad_tokens")):
        assert (buf.cpu()[mask] == -3.0).all(), f"padding of {what} was written"


# ------------------------------------------------------------------ tiled path (persistent
# grid, decoupled look-back), called through the C ABI so the workspace can be inspected
def _abi():
    import ctypes
    import os

    lib = ctypes.CDLL(os.path.join(os.path.dirname(fpscan_amd.__file__), "libfpscan_hip.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_scan_fwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                    ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fpscan_scan_bwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                    vp, ctypes.c_size_t, vp]
    lib.fpscan_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int, ctypes.c_int]
    lib.fpscan_workspace_bytes.restype = ctypes.c_size_t
    lib.fpscan_set_tiling.argtypes = [ctypes.c_int]
    return lib


_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _abi_scan(lib, g, x, reverse, tiled):
    B, D, L = x.shape
    out = torch.empty_like(x)
    nbytes = lib.fpscan_workspace_bytes(B, D, L, _CODE[x.dtype], 0) if tiled else 0
    ws = torch.full((max(nbytes, 8),), 0xA5, dtype=torch.uint8, device=DEVICE)  # stale data
    st = lib.fpscan_scan_fwd(g.data_ptr(), x.data_ptr(), out.data_ptr(), B, D, L, D * L, L,
                             _CODE[x.dtype], int(reverse), ws.data_ptr() if nbytes else None,
                             nbytes, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    return out, ws, nbytes


def _abi_bwd(lib, g, y, go, tiled):
    B, D, L = g.shape
    gg, gx = torch.empty_like(g), torch.empty_like(g)
    nbytes = lib.fpscan_workspace_bytes(B, D, L, _CODE[g.dtype], 1) if tiled else 0
    ws = torch.full((max(nbytes, 8),), 0xA5, dtype=torch.uint8, device=DEVICE)  # stale data
    st = lib.fpscan_scan_bwd(g.data_ptr(), y.data_ptr(), go.data_ptr(), gg.data_ptr(),
                             gx.data_ptr(), B, D, L, D * L, L, _CODE[g.dtype],
                             ws.data_ptr() if nbytes else None, nbytes,
                             torch.cuda.current_stream().cuda_stream)
    assert st == 0
    return gg, gx, ws, nbytes


CLAIM_GROUPS, COUNTER_STRIDE = 8, 16  # workspace tail: overrun word, then 8 claim counters


def _overruns(ws, nbytes):
    """The word after the tile status words counts look-back waits that hit their bound (0 in
    a good run). Every tile must have been published, and the claim counters must have handed
    out at least every tile."""
    words = ws[:nbytes].view(torch.int64)
    ntiles = nbytes // 8 - COUNTER_STRIDE * (1 + CLAIM_GROUPS)
    counters = words[ntiles + COUNTER_STRIDE::COUNTER_STRIDE]
    assert counters.numel() == CLAIM_GROUPS
    assert int(counters.sum().item()) >= ntiles, "not every tile was claimed"
    assert (words[:ntiles] != -1).all(), "a tile was never published"
    return int(words[ntiles].item())


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", [(1, 3, 8192), (2, 8, 16384), (3, 5, 65536), (32, 64, 8192)])
def test_tiled_path_matches_oracle(dtype, shape):
    """Shapes from one tile per row (fp16/bf16 at 8192) to 64 tiles per row (fp32 at 65536)."""
    lib = _abi()
    lib.fpscan_set_tiling(2)
    try:
        g, x = make_inputs(*shape, dtype, seed=sum(shape))
        gd, xd = g.to(DEVICE), x.to(DEVICE)
        for rev in (False, True):
            out, ws, nbytes = _abi_scan(lib, gd, xd, rev, tiled=True)
            assert nbytes > 0
            torch.cuda.synchronize()
            assert _overruns(ws, nbytes) == 0
            check(out, oracle.scan_f64(g, x, rev), dtype, f"tiled rev={rev}")
        go = torch.randn(g.shape, generator=torch.Generator().manual_seed(8)).to(dtype)
        y = fpscan_amd.scan_forward(gd, xd)
        gg, gx, ws, nbytes = _abi_bwd(lib, gd, y, go.to(DEVICE), tiled=True)
        torch.cuda.synchronize()
        assert _overruns(ws, nbytes) == 0
        gg_ref, gx_ref = oracle.scan_bwd_f64(g, y.cpu(), go)
        check(gx, gx_ref, dtype, "tiled grad_tokens")
        check(gg, gg_ref, dtype, "tiled grad_gates")
    finally:
        lib.fpscan_set_tiling(0)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_tiled_path_exact_on_integer_data(dtype):
    lib = _abi()
    lib.fpscan_set_tiling(2)
    try:
        gen = torch.Generator().manual_seed(99)
        L = 65536
        gi = (torch.randint(0, 16, (2, 3, L), generator=gen) > 0).to(dtype)
        xi = torch.randint(-3, 4, (2, 3, L), generator=gen).to(dtype)
        for rev in (False, True):
            out, ws, nbytes = _abi_scan(lib, gi.to(DEVICE), xi.to(DEVICE), rev, tiled=True)
            want = torch.from_numpy(oracle.scan_f64(gi, xi, rev))
            if dtype == torch.float32 or want.abs().max() < 256:
                assert bits_equal(out.cpu(), want.to(dtype))
            assert _overruns(ws, nbytes) == 0
    finally:
        lib.fpscan_set_tiling(0)


def test_tiled_and_streaming_paths_agree_and_default_is_tiled_when_large():
    lib = _abi()
    g, x, go = _bench_inputs(8, 1024, 65536, torch.bfloat16, "mamba", seed=6)  # 1 GiB each
    assert lib.fpscan_workspace_bytes(8, 1024, 65536, 2, 0) > 0  # tiled by default at this size
    assert lib.fpscan_workspace_bytes(2, 512, 65536, 2, 0) == 0  # 64 MiB: rows are streamed
    tiled, ws, nbytes = _abi_scan(lib, g, x, False, tiled=True)
    streamed, _, _ = _abi_scan(lib, g, x, False, tiled=False)
    torch.cuda.synchronize()
    assert _overruns(ws, nbytes) == 0
    assert oracle.normwise_error(tiled, streamed) < 2e-2
    rows = torch.linspace(0, 8191, 16).long()
    gs, xs = g.reshape(8192, -1)[rows].cpu(), x.reshape(8192, -1)[rows].cpu()
    check(tiled.reshape(8192, -1)[rows], oracle.scan_f64(gs, xs), torch.bfloat16, "tiled c4")


@pytest.mark.parametrize("B,L", [(2, 65536), (4, 32768)], ids=["rows128k", "rows64k"])
def test_backward_tiles_long_rows_from_256_mib(B, L):
    """bf16 (B, 1024, L) at 256 MiB per tensor with rows of 128 KiB and 64 KiB: the automatic
    plan tiles the backward but streams the forward. The automatic backward agrees with the
    streamed one and with the oracle on sampled rows."""
    lib = _abi()
    assert lib.fpscan_workspace_bytes(B, 1024, L, 2, 1) > 0
    assert lib.fpscan_workspace_bytes(B, 1024, L, 2, 0) == 0
    g, x, go = _bench_inputs(B, 1024, L, torch.bfloat16, "mamba", seed=8)
    y = fpscan_amd.scan_forward(g, x)
    gg, gx = fpscan_amd.scan_backward(g, y, go)  # automatic: tiled
    try:
        ops.set_tiling(1)
        gg_s, gx_s = fpscan_amd.scan_backward(g, y, go)
    finally:
        ops.set_tiling(0)
    torch.cuda.synchronize()
    assert oracle.normwise_error(gx, gx_s) < 2e-2
    assert oracle.normwise_error(gg, gg_s) < 2e-2
    nrows = B * 1024
    rows = torch.linspace(0, nrows - 1, 8).long()
    gs = g.reshape(nrows, -1)[rows].cpu()
    ys, gos = y.reshape(nrows, -1)[rows].cpu(), go.reshape(nrows, -1)[rows].cpu()
    gg_ref, gx_ref = oracle.scan_bwd_f64(gs, ys, gos)
    check(gx.reshape(nrows, -1)[rows], gx_ref, torch.bfloat16, "tiled bwd 256 MiB grad_tokens")
    check(gg.reshape(nrows, -1)[rows], gg_ref, torch.bfloat16, "tiled bwd 256 MiB grad_gates")


# ------------------------------------------------------------------ padded strides (C ABI)
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("L", [64, 4096, 65536])
@pytest.mark.parametrize("tiled", [False, True], ids=["stream", "tiled"])
def test_padded_strides_through_the_c_abi(dtype, L, tiled):
    """Rows of a larger buffer: stride_d = L + pad, stride_b = dim * stride_d + pad2. Only
    the (batch, dim, seqlen) view may change; the padding must come back untouched."""
    lib = _abi()
    B, D = 2, 3
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    sd = L + 8 * vec
    sb = D * sd + 4 * vec
    g, x = make_inputs(B, D, L, dtype, seed=L + tiled)
    go = torch.randn(B, D, L, generator=torch.Generator().manual_seed(1)).to(dtype)

    def embed(t, fill):
        buf = torch.full((B * sb,), fill, dtype=dtype)
        view = buf.as_strided((B, D, L), (sb, sd, 1))
        view.copy_(t)
        return buf.to(DEVICE)

    def view(buf):
        return buf.as_strided((B, D, L), (sb, sd, 1))

    gb, xb, gob = embed(g, 7.0), embed(x, 7.0), embed(go, 7.0)
    outb, ggb, gxb = embed(torch.zeros_like(x), -3.0), embed(torch.zeros_like(x), -3.0), \
        embed(torch.zeros_like(x), -3.0)
    lib.fpscan_set_tiling(2 if tiled else 1)
    try:
        stream = torch.cuda.current_stream().cuda_stream
        code = _CODE[dtype]
        nb = lib.fpscan_workspace_bytes(B, D, L, code, 0) if tiled else 0
        ws = torch.empty(max(nb, 8), dtype=torch.uint8, device=DEVICE)
        assert lib.fpscan_scan_fwd(gb.data_ptr(), xb.data_ptr(), outb.data_ptr(), B, D, L, sb, sd,
                                   code, 0, ws.data_ptr() if nb else None, nb, stream) == 0
        nb = lib.fpscan_workspace_bytes(B, D, L, code, 1) if tiled else 0
        ws = torch.empty(max(nb, 8), dtype=torch.uint8, device=DEVICE)
        assert lib.fpscan_scan_bwd(gb.data_ptr(), outb.data_ptr(), gob.data_ptr(), ggb.data_ptr(),
                                   gxb.data_ptr(), B, D, L, sb, sd, code,
                                   ws.data_ptr() if nb else None, nb, stream) == 0
        torch.cuda.synchronize()
    finally:
        lib.fpscan_set_tiling(0)
    out = view(outb).cpu()
    check(out, oracle.scan_f64(g, x), dtype, f"strided fwd L{L}")
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, out, go)
    check(view(gxb).cpu(), gx_ref, dtype, f"strided grad_tokens L{L}")
    check(view(ggb).cpu(), gg_ref, dtype, f"strided grad_gates L{L}")
    mask = torch.ones(B * sb, dtype=torch.bool)
    mask.as_strided((B, D, L), (sb, sd, 1)).fill_(False)
    for buf in (outb, ggb, gxb):
        assert (buf.cpu()[mask] == -3.0).all(), "padding was written"


# ------------------------------------------------------------------ HIP graph capture
# Kept skipped: its one run (the streaming case) ended with a host segmentation fault inside
# torch.cuda.graph's capture_end (graph instantiation), with a cause not identified. The
# torch binding now refuses capture before any launch (test_robustness_gpu.py checks that),
# so this test would fail at the refusal until capture is supported again.
@pytest.mark.skip(reason="the host process ended with a segmentation fault inside "
                         "torch.cuda.graph's capture_end on the first (streaming) case; the "
                         "cause is not identified, so the case stays off the GPU and the "
                         "binding refuses capture")
@pytest.mark.parametrize("shape", [(2, 4, 1024), (8, 1024, 65536)], ids=["stream", "tiled"])
def test_graph_capture_replays_match_eager(shape):
    """pscan forward + backward captured in a HIP graph (the tiled path's status clear is a
    kernel, its workspace comes from the graph's pool) and replayed several times with eager
    work in between; every replay must equal the eager result bit for bit."""
    import bench

    dtype = torch.bfloat16
    g, x, go = bench.make_inputs(*shape, dtype, "mamba", seed=12, device=DEVICE)
    gr = g.clone().requires_grad_()
    xr = x.clone().requires_grad_()

    def step():
        y = fpscan_amd.pscan(gr, xr)
        gg, gx = torch.autograd.grad(y, (gr, xr), go)
        return y, gg, gx

    want = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = step()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert bits_equal(a, b), f"replay {i} differs"
        fpscan_amd.scan_forward(g, x)  # eager work between replays
        torch.cuda.synchronize()
