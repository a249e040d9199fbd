"""GPU parity tests of the fused gate producer: the scan with gates exp(-softplus(z) * rate[d])
computed inside the kernels (pscan_softplus, scan_forward_softplus, scan_backward_softplus),
against the float64 oracle (oracle.scan_softplus_f64 / scan_bwd_softplus_f64, pinned in
tests/test_oracle.py by float64 autograd through torch's softplus and exp), and against the
unfused composition it replaces (torch computes the gates, then the scan)."""
import numpy as np
import pytest
import torch

import fpscan_amd
import oracle
from scan_helpers import ALL_SEQLENS, DEVICE, DTYPES, NORM_TOL, bits_equal, check

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]


def sp_inputs(B, D, L, dtype, seed=0):
    """Mamba-like: z = N(0, 1) (delta = softplus(z)), rate in [0.001, 0.1] so that the gates
    (around 0.95-1) carry state over many steps; tokens 0.1 N(0, 1)."""
    gen = torch.Generator().manual_seed(seed)
    z = torch.randn(B, D, L, generator=gen).to(dtype)
    rate = 0.001 + 0.099 * torch.rand(D, generator=gen)
    x = (0.1 * torch.randn(B, D, L, generator=gen)).to(dtype)
    return z, rate, x


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", ALL_SEQLENS)
def test_forward_and_reverse_match_oracle(dtype, seqlen):
    z, rate, x = sp_inputs(2, 4, seqlen, dtype, seed=seqlen)
    zd, rd, xd = z.to(DEVICE), rate.to(DEVICE), x.to(DEVICE)
    for rev in (False, True):
        out = fpscan_amd.scan_forward_softplus(zd, rd, xd, reverse=rev)
        check(out, oracle.scan_softplus_f64(z, rate, x, rev), dtype, f"softplus L{seqlen} rev={rev}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("seqlen", [32, 256, 512, 4096, 65536])
def test_backward_matches_oracle(dtype, seqlen):
    z, rate, x = sp_inputs(3, 5, seqlen, dtype, seed=seqlen + 1)
    go = torch.randn(z.shape, generator=torch.Generator().manual_seed(2)).to(dtype)
    zd, rd = z.to(DEVICE), rate.to(DEVICE)
    y = fpscan_amd.scan_forward_softplus(zd, rd, x.to(DEVICE))
    gz, gr, gx = fpscan_amd.scan_backward_softplus(zd, rd, y, go.to(DEVICE))
    gz_ref, gr_ref, gx_ref = oracle.scan_bwd_softplus_f64(z, rate, y.cpu(), go)
    check(gx, gx_ref, dtype, f"grad_tokens L{seqlen}")
    check(gz, gz_ref, dtype, f"grad_z L{seqlen}")
    assert gr.dtype == torch.float32 and gr.shape == rate.shape
    # grad_rate sums N-length products in fp32; the bar is the fp32 one scaled by the row count
    err = oracle.normwise_error(gr, gr_ref)
    assert err <= max(NORM_TOL[dtype], 1e-4), f"grad_rate L{seqlen}: {err:.3e}"


@pytest.mark.parametrize("z_mean", [-9.0, -18.0])
@pytest.mark.parametrize("seqlen", [128, 4096, 65536])
def test_small_delta_channels_keep_grad_rate_accurate(z_mean, seqlen):
    """Channels with a small step size (z well below 0, softplus(z) ~ exp(z)): the gate's
    exponent softplus(z) * rate and d gate / d rate = -gate * softplus(z) need softplus to
    relative accuracy where 1 + exp(z) rounds to nearly (z = -9) or exactly (z = -18) 1 in
    fp32. The rates are scaled by exp(-z_mean) so that the gates decay (about 0.99 per step)
    instead of summing thousands of steps, whose fp32 accumulation alone nears 1e-5. Outputs,
    grad_rate, grad_z and grad_tokens must meet the fp32 bar against the float64 oracle on
    short rows, streamed rows and long rows."""
    gen = torch.Generator().manual_seed(int(-z_mean) * 100 + seqlen)
    B, D = 2, 6
    z = torch.randn(B, D, seqlen, generator=gen) + z_mean
    rate = 0.01 * float(np.exp(-z_mean)) * (0.5 + 1.5 * torch.rand(D, generator=gen))
    x = 0.1 * torch.randn(B, D, seqlen, generator=gen)
    go = torch.randn(B, D, seqlen, generator=gen)
    zd, rd = z.to(DEVICE), rate.to(DEVICE)
    y = fpscan_amd.scan_forward_softplus(zd, rd, x.to(DEVICE))
    check(y, oracle.scan_softplus_f64(z, rate, x), torch.float32, f"y z~N({z_mean},1)")
    gz, gr, gx = fpscan_amd.scan_backward_softplus(zd, rd, y, go.to(DEVICE))
    gz_ref, gr_ref, gx_ref = oracle.scan_bwd_softplus_f64(z, rate, y.cpu(), go)
    check(gx, gx_ref, torch.float32, f"grad_tokens z~N({z_mean},1)")
    check(gz, gz_ref, torch.float32, f"grad_z z~N({z_mean},1)")
    err = oracle.normwise_error(gr, gr_ref)
    assert err <= NORM_TOL[torch.float32], f"grad_rate z~N({z_mean},1) L{seqlen}: {err:.3e}"


@pytest.mark.parametrize("dtype,L", [(torch.bfloat16, 8192), (torch.float32, 16384)], ids=str)
def test_short_rows_of_16_to_64_mib_match_oracle(dtype, L):
    """1024 rows of 16 (bf16) or 64 (fp32) sub-chunks, 16-64 MiB per tensor: shapes that
    stream as 8-wave rows by default, forward and backward; sampled rows against the oracle,
    every row against the 16-wave launch."""
    z, rate, x = sp_inputs(1, 1024, L, dtype, seed=L)
    go = torch.randn(z.shape, generator=torch.Generator().manual_seed(6)).to(dtype)
    zd, rd, xd, god = z.to(DEVICE), rate.to(DEVICE), x.to(DEVICE), go.to(DEVICE)
    y = fpscan_amd.scan_forward_softplus(zd, rd, xd)
    gz, gr, gx = fpscan_amd.scan_backward_softplus(zd, rd, y, god)
    rows = [0, 1, 511, 1022, 1023]
    sel = lambda t: t.reshape(1024, L)[rows].reshape(1, len(rows), L).cpu()  # noqa: E731
    check(sel(y), oracle.scan_softplus_f64(sel(z), rate[rows], sel(x)), dtype, "short rows y")
    gz_ref, gr_ref, gx_ref = oracle.scan_bwd_softplus_f64(sel(z), rate[rows], sel(y), sel(go))
    check(sel(gx), gx_ref, dtype, "short rows grad_tokens")
    check(sel(gz), gz_ref, dtype, "short rows grad_z")
    assert oracle.normwise_error(gr[rows], gr_ref) <= max(NORM_TOL[dtype], 1e-4)
    try:
        fpscan_amd.ops.set_launch_override(16, 0)
        y16 = fpscan_amd.scan_forward_softplus(zd, rd, xd)
        gz16, gr16, gx16 = fpscan_amd.scan_backward_softplus(zd, rd, y, god)
    finally:
        fpscan_amd.ops.set_launch_override(0, 0)
    for got, want, what in ((y, y16, "y"), (gx, gx16, "grad_tokens"), (gz, gz16, "grad_z"),
                            (gr, gr16, "grad_rate")):
        assert oracle.normwise_error(got, want) <= max(NORM_TOL[dtype], 1e-5), what


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_one_row_per_block_matches_oracle_and_four_rows_per_block(dtype):
    """65578 rows of one sub-chunk: each row a 64-thread block of its own, forward and
    backward; sampled rows against the oracle, every output bit for bit against the
    4-rows-per-block launch that a launch override selects."""
    L = 256 if dtype == torch.float32 else 512
    B, D = 2, 32768 + 21
    z, rate, x = sp_inputs(B, D, L, dtype, seed=L + 3)
    go = torch.randn(z.shape, generator=torch.Generator().manual_seed(7)).to(dtype)
    zd, rd, xd, god = z.to(DEVICE), rate.to(DEVICE), x.to(DEVICE), go.to(DEVICE)
    y = fpscan_amd.scan_forward_softplus(zd, rd, xd)
    gz, gr, gx = fpscan_amd.scan_backward_softplus(zd, rd, y, god)
    try:
        fpscan_amd.ops.set_launch_override(1, 1)
        y4 = fpscan_amd.scan_forward_softplus(zd, rd, xd)
        gz4, gr4, gx4 = fpscan_amd.scan_backward_softplus(zd, rd, y, god)
    finally:
        fpscan_amd.ops.set_launch_override(0, 0)
    for got, want, what in ((y, y4, "y"), (gz, gz4, "grad_z"), (gx, gx4, "grad_tokens"),
                            (gr, gr4, "grad_rate")):
        assert bits_equal(got, want), f"{what}: one row per block differs from four"
    rows = [0, 1, D - 1, D, 2 * D - 1]
    sel = lambda t: t.reshape(B * D, L)[rows].reshape(1, len(rows), L).cpu()  # noqa: E731
    rsel = rate[[r % D for r in rows]]
    check(sel(y), oracle.scan_softplus_f64(sel(z), rsel, sel(x)), dtype, "one-row blocks y")
    gz_ref, _, gx_ref = oracle.scan_bwd_softplus_f64(sel(z), rsel, sel(y), sel(go))
    check(sel(gx), gx_ref, dtype, "one-row blocks grad_tokens")
    check(sel(gz), gz_ref, dtype, "one-row blocks grad_z")


@pytest.mark.parametrize("seqlen", [64, 1024, 65536])
def test_equals_the_unfused_composition(seqlen):
    """fp32: torch computes the gates, then the scan; the fused kernels must agree to fp32
    rounding (the only difference is how exp and log are evaluated)."""
    z, rate, x = sp_inputs(2, 8, seqlen, torch.float32, seed=5)
    zd, rd, xd = z.to(DEVICE), rate.to(DEVICE), x.to(DEVICE)
    gates = torch.exp(-torch.nn.functional.softplus(zd) * rd[None, :, None])
    want = fpscan_amd.scan_forward(gates.contiguous(), xd)
    got = fpscan_amd.scan_forward_softplus(zd, rd, xd)
    assert oracle.normwise_error(got, want) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_autograd_matches_oracle(dtype):
    z, rate, x = sp_inputs(2, 6, 8192, dtype, seed=9)
    go = torch.randn(z.shape, generator=torch.Generator().manual_seed(3)).to(dtype)
    zd = z.to(DEVICE).requires_grad_()
    rd = rate.to(DEVICE).requires_grad_()
    xd = x.to(DEVICE).requires_grad_()
    y = fpscan_amd.pscan_softplus(zd, rd, xd)
    y.backward(go.to(DEVICE))
    check(y, oracle.scan_softplus_f64(z, rate, x), dtype, "autograd y")
    gz_ref, gr_ref, gx_ref = oracle.scan_bwd_softplus_f64(z, rate, y.detach().cpu(), go)
    check(xd.grad, gx_ref, dtype, "autograd grad_tokens")
    check(zd.grad, gz_ref, dtype, "autograd grad_z")
    assert oracle.normwise_error(rd.grad, gr_ref) <= max(NORM_TOL[dtype], 1e-4)


def test_extreme_z_saturates():
    """z -> -inf gives gate 1 (cumsum), z -> +inf gives gate 0 (y = x)."""
    x = torch.randn(1, 2, 1024, device=DEVICE)
    rate = torch.ones(2, device=DEVICE)
    lo = fpscan_amd.scan_forward_softplus(torch.full_like(x, -200.0), rate, x)
    torch.testing.assert_close(lo, torch.cumsum(x, -1), rtol=1e-5, atol=1e-4)
    hi = fpscan_amd.scan_forward_softplus(torch.full_like(x, 200.0), rate, x)
    assert torch.equal(hi, x)


def test_validation_errors():
    z = torch.randn(2, 3, 64, device=DEVICE)
    r = torch.rand(3, device=DEVICE)
    with pytest.raises(RuntimeError, match="float32"):
        fpscan_amd.scan_forward_softplus(z, r.half(), z)
    with pytest.raises(RuntimeError, match="one value per dim"):
        fpscan_amd.scan_forward_softplus(z, r[:2].contiguous(), z)
    with pytest.raises(RuntimeError, match="seqlen"):
        fpscan_amd.scan_forward_softplus(z[..., :48].contiguous(), r, z[..., :48].contiguous())
    with pytest.raises(RuntimeError, match="dtype"):
        fpscan_amd.scan_forward_softplus(z.half(), r, z)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_headline_shape_b8_d1024_l65536(dtype):
    gen = torch.Generator(device=DEVICE).manual_seed(4)
    B, D, L = 8, 1024, 65536
    z = torch.randn(B, D, L, generator=gen, device=DEVICE).to(dtype)
    rate = 0.001 + 0.099 * torch.rand(D, generator=gen, device=DEVICE)
    x = (0.1 * torch.randn(B, D, L, generator=gen, device=DEVICE)).to(dtype)
    go = torch.randn(B, D, L, generator=gen, device=DEVICE).to(dtype)
    y = fpscan_amd.scan_forward_softplus(z, rate, x)
    gz, gr, gx = fpscan_amd.scan_backward_softplus(z, rate, y, go)
    rows = [0, 5, 1023, 4099, 8191]
    sel = lambda t: t.reshape(B * D, L)[rows].reshape(1, len(rows), L).cpu()  # noqa: E731
    rsel = rate.cpu()[[r % D for r in rows]]
    check(sel(y), oracle.scan_softplus_f64(sel(z), rsel, sel(x)), dtype, "headline y")
    gz_ref, _, gx_ref = oracle.scan_bwd_softplus_f64(sel(z), rsel, sel(y), sel(go))
    check(sel(gx), gx_ref, dtype, "headline grad_tokens")
    check(sel(gz), gz_ref, dtype, "headline grad_z")
    assert torch.isfinite(gr).all()
