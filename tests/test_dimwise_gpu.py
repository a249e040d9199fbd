"""GPU parity tests of dimwise_forward (the reference module's contraction scan,
csrc/main.cpp:10, csrc/dimwise/) against the float64 oracle (oracle.dimwise_f64, pinned in
tests/test_oracle.py by a restatement of the reference's own Python model).

The reference's only check of this function is scans/contraction_scan.py:144-185 (fp32,
atol 1e-3 against its Python model); here every supported seqlen runs in every dtype, with
the north-star normwise tolerances. The selection (a first maximum) is discontinuous, so the
half-precision cases draw keys that are well apart and group sums of one sign: the same group
is then chosen in any precision, as it must be for results to agree at all.
"""
import numpy as np
import pytest
import torch

import fpscan_amd
import oracle
from fpscan_amd import ops
from scan_helpers import DEVICE, DTYPES, check

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]

SEQLENS = sorted(oracle.DIMWISE_GEOMETRY)
# seqlens with two or more chunks of 32 groups of 128, where the tiled path applies
TILED_SEQLENS = [L for L in SEQLENS if L >= 8192]


class tiling:
    """Path selection for the duration of a block: 1 row kernel only, 2 tiled when the
    seqlen allows (fpscan_set_tiling)."""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        ops.set_tiling(self.mode)

    def __exit__(self, *exc):
        ops.set_tiling(0)


def driver_inputs(B, D, L, seed=0):
    """scans/contraction_scan.py:154-159: Ax 0.99 + 0.01 U, Bx N/G, Bh N/G, Wq/Wk 0.01 U."""
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    G = W * C
    gen = torch.Generator().manual_seed(seed)
    ax = 0.99 + 0.01 * torch.rand(B, D, L, generator=gen)
    bx = torch.randn(B, D, L, generator=gen) / G
    bh = torch.randn(B, D, G, generator=gen) / G
    wq = 0.01 * torch.rand(D, generator=gen)
    wk = 0.01 * torch.rand(D, generator=gen)
    return ax, bx, bh, wq, wk


def separated_inputs(B, D, L, sign=1.0, seed=0):
    """Keys a permutation of evenly spaced values per row (about 6 % apart), tokens of one
    sign (so every q has that sign): the selection is unambiguous in fp16 and bf16 too."""
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    G = W * C
    gen = torch.Generator().manual_seed(seed)
    ax = 0.99 + 0.01 * torch.rand(B, D, L, generator=gen)
    bx = sign * (0.5 + 0.5 * torch.rand(B, D, L, generator=gen)) / P
    ranks = torch.rand(B, D, W, generator=gen).argsort(dim=-1).argsort(dim=-1).double()
    bh = torch.randn(B, D, G, generator=gen) / G
    bh[:, :, :W] = (-1.0 + 2.0 * ranks / max(W - 1, 1)) / 4
    wq = 0.01 * torch.rand(D, generator=gen)
    wk = 0.01 * torch.rand(D, generator=gen)
    return ax, bx, bh.float(), wq, wk


def run(ax, bx, bh, wq, wk, dtype):
    t = [v.to(dtype).contiguous() for v in (ax, bx, bh, wq, wk)]
    want = oracle.dimwise_f64(*t)
    dev = [v.to(DEVICE) for v in t]
    assert fpscan_amd.dimwise_forward(*dev) is None  # in place, returns nothing
    return dev[1], want


@pytest.mark.parametrize("L", SEQLENS)
def test_fp32_driver_distribution_matches_oracle(L):
    got, want = run(*driver_inputs(2, 4, L, seed=L), torch.float32)
    check(got, want, torch.float32, f"dimwise fp32 L{L}")
    # the reference's own bar (scans/contraction_scan.py:184)
    assert np.abs(got.double().cpu().numpy() - want).max() < 1e-3


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("L", SEQLENS)
@pytest.mark.parametrize("sign", [1.0, -1.0], ids=["q>0", "q<0"])
def test_separated_keys_match_oracle(L, dtype, sign):
    got, want = run(*separated_inputs(2, 3, L, sign=sign, seed=L + 7), dtype)
    check(got, want, dtype, f"dimwise {dtype} L{L} sign {sign}")


@pytest.mark.parametrize("L", [64, 4096, 16384])
def test_unit_gates_zero_keys_exact(L):
    """Gates 1, k = 0, integer tokens: every partial result is an exact integer, so the
    output must equal the oracle bit for bit (group cumsums plus the previous group's total,
    group 0 continuing from the chunk carry)."""
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    gen = torch.Generator().manual_seed(L)
    x = torch.randint(-4, 5, (2, 3, L), generator=gen).float()
    ones = torch.ones_like(x)
    got, want = run(ones, x, torch.zeros(2, 3, W * C), torch.zeros(3), torch.zeros(3),
                    torch.float32)
    assert torch.equal(got.cpu().double(), torch.from_numpy(want))


def test_first_gate_is_ignored():
    ax, bx, bh, wq, wk = driver_inputs(1, 2, 4096, seed=3)
    axn = ax.clone()
    axn[:, :, 0] = float("nan")
    got, _ = run(axn, bx, bh, wq, wk, torch.float32)
    ref, _ = run(ax, bx, bh, wq, wk, torch.float32)
    assert torch.equal(got, ref)


def test_shapes_and_rows():
    """Ragged row counts and a single row."""
    for B, D in [(1, 1), (3, 5), (7, 33)]:
        got, want = run(*driver_inputs(B, D, 8192, seed=B * D), torch.float32)
        check(got, want, torch.float32, f"dimwise B{B} D{D}")


def test_empty_and_validation():
    x = torch.rand(2, 3, 64, device=DEVICE)
    bh = torch.rand(2, 3, 2, device=DEVICE)
    w = torch.rand(3, device=DEVICE)
    fpscan_amd.dimwise_forward(x[:0], x[:0].clone(), bh[:0], w, w)  # empty: nothing to do
    for L in (32, 96, 131072):
        y = torch.rand(1, 1, L, device=DEVICE)
        with pytest.raises(RuntimeError, match="seqlen"):
            fpscan_amd.dimwise_forward(y, y.clone(), torch.rand(1, 1, 2, device=DEVICE),
                                       w[:1], w[:1])
    with pytest.raises(RuntimeError, match="Bh must have shape"):
        fpscan_amd.dimwise_forward(x, x.clone(), torch.rand(2, 3, 4, device=DEVICE), w, w)
    with pytest.raises(RuntimeError, match="Wq and Wk"):
        fpscan_amd.dimwise_forward(x, x.clone(), bh, w[:2], w)
    with pytest.raises(RuntimeError, match="dtype"):
        fpscan_amd.dimwise_forward(x, x.clone(), bh.half(), w, w)
    with pytest.raises(RuntimeError, match="contiguous"):
        fpscan_amd.dimwise_forward(x, x.clone().transpose(0, 1), bh, w, w)
    with pytest.raises(RuntimeError, match="CUDA"):
        fpscan_amd.dimwise_forward(x.cpu(), x.clone(), bh, w, w)
    # Bx is written in place: Ax may be Bx itself but not part of it, and the per-row
    # parameters must not lie inside it
    buf = torch.rand(2 * 3 * 64 + 64, device=DEVICE)
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.dimwise_forward(buf[64:].view(2, 3, 64), buf[:-64].view(2, 3, 64), bh, w, w)
    bx = x.clone()
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.dimwise_forward(x, bx, bh, bx.view(-1)[:3], w)
    assert fpscan_amd.dimwise_groups(65536) == 512 and fpscan_amd.dimwise_groups(32) == 0


# ------------------------------------------------------------------ tiled path
@pytest.mark.parametrize("L", TILED_SEQLENS)
def test_tiled_fp32_driver_distribution_matches_oracle(L):
    with tiling(2):
        got, want = run(*driver_inputs(2, 4, L, seed=L), torch.float32)
    check(got, want, torch.float32, f"dimwise tiled fp32 L{L}")
    assert np.abs(got.double().cpu().numpy() - want).max() < 1e-3


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("L", TILED_SEQLENS)
@pytest.mark.parametrize("sign", [1.0, -1.0], ids=["q>0", "q<0"])
def test_tiled_separated_keys_match_oracle(L, dtype, sign):
    with tiling(2):
        got, want = run(*separated_inputs(2, 3, L, sign=sign, seed=L + 7), dtype)
    check(got, want, dtype, f"dimwise tiled {dtype} L{L} sign {sign}")


@pytest.mark.parametrize("L", [8192, 16384, 65536])
def test_tiled_unit_gates_zero_keys_exact(L):
    """As test_unit_gates_zero_keys_exact on the tiled path: the carry maps composed across
    tiles are exact on integers too, so the output equals the oracle bit for bit."""
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    gen = torch.Generator().manual_seed(L + 1)
    x = torch.randint(-4, 5, (2, 3, L), generator=gen).float()
    ones = torch.ones_like(x)
    with tiling(2):
        got, want = run(ones, x, torch.zeros(2, 3, W * C), torch.zeros(3), torch.zeros(3),
                        torch.float32)
    assert torch.equal(got.cpu().double(), torch.from_numpy(want))


def test_tiled_first_gate_is_ignored():
    ax, bx, bh, wq, wk = driver_inputs(1, 2, 16384, seed=4)
    axn = ax.clone()
    axn[:, :, 0] = float("nan")
    with tiling(2):
        got, _ = run(axn, bx, bh, wq, wk, torch.float32)
        ref, _ = run(ax, bx, bh, wq, wk, torch.float32)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("L", [8192, 32768])
def test_tiled_shapes_and_rows(L):
    """Ragged row counts and a single row; at 8192 a bf16 row is one tile (no look-back),
    an fp32 row two."""
    for B, D in [(1, 1), (3, 5), (7, 33)]:
        for dtype in (torch.float32, torch.bfloat16):
            with tiling(2):
                got, want = run(*separated_inputs(B, D, L, seed=B * D + L), dtype)
            check(got, want, dtype, f"dimwise tiled {dtype} B{B} D{D} L{L}")


@pytest.mark.parametrize("mode", [1, 2], ids=["rows", "tiled"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_headline_shape_b8_d1024_l65536(dtype, mode):
    """The headline shape on each path: sampled rows against the oracle (all rows run on the
    GPU)."""
    gen = torch.Generator(device=DEVICE).manual_seed(11)
    B, D, L = 8, 1024, 65536
    ax = (0.99 + 0.01 * torch.rand(B, D, L, generator=gen, device=DEVICE)).to(dtype)
    bx = ((0.5 + 0.5 * torch.rand(B, D, L, generator=gen, device=DEVICE)) / 128).to(dtype)
    ranks = torch.rand(B, D, 32, generator=gen, device=DEVICE).argsort(-1).argsort(-1).float()
    bh = torch.randn(B, D, 512, generator=gen, device=DEVICE) / 512
    bh[:, :, :32] = (-1.0 + 2.0 * ranks / 31) / 4
    bh = bh.to(dtype)
    wq = (0.01 * torch.rand(D, generator=gen, device=DEVICE)).to(dtype)
    wk = (0.01 * torch.rand(D, generator=gen, device=DEVICE)).to(dtype)
    rows = [0, 1, 1023, 4096, 8191]
    sel = lambda t: t.reshape(B * D, -1)[rows].reshape(1, len(rows), -1).cpu()  # noqa: E731
    want = oracle.dimwise_f64(sel(ax), sel(bx), sel(bh), wq.cpu()[[r % D for r in rows]],
                              wk.cpu()[[r % D for r in rows]])
    before = fpscan_amd.lookback_overruns()
    with tiling(mode):
        fpscan_amd.dimwise_forward(ax, bx, bh, wq, wk)
    check(sel(bx), want, dtype, f"dimwise headline {dtype} tiling {mode}")
    assert fpscan_amd.lookback_overruns() == before


@pytest.mark.parametrize("B", [15, 16], ids=["3.75GiB-tiled", "4GiB-rows"])
def test_tensors_near_4_gib(B):
    """fp32 (B, 1024, 65536): 3.75 GiB per tensor takes the tiled path, whose tile offsets are
    32-bit byte offsets into one buffer range per tensor; 4 GiB takes the row kernel. Sampled
    rows, the last ones included, against the oracle."""
    D, L = 1024, 65536
    tiled = ops.dimwise_workspace_bytes(B, D, L, torch.float32) > 0
    assert tiled == (B * D * L * 4 < (1 << 32))
    gen = torch.Generator(device=DEVICE).manual_seed(B)
    ax = 0.99 + 0.01 * torch.rand(B, D, L, generator=gen, device=DEVICE)
    bx = (0.5 + 0.5 * torch.rand(B, D, L, generator=gen, device=DEVICE)) / 128
    bh = torch.randn(B, D, 512, generator=gen, device=DEVICE) / 512
    wq = 0.01 * torch.rand(D, generator=gen, device=DEVICE)
    wk = 0.01 * torch.rand(D, generator=gen, device=DEVICE)
    rows = [0, 1, B * D // 2, B * D - 2, B * D - 1]
    sel = lambda t: t.reshape(B * D, -1)[rows].reshape(1, len(rows), -1).cpu()  # noqa: E731
    want = oracle.dimwise_f64(sel(ax), sel(bx), sel(bh), wq.cpu()[[r % D for r in rows]],
                              wk.cpu()[[r % D for r in rows]])
    before = fpscan_amd.lookback_overruns()
    fpscan_amd.dimwise_forward(ax, bx, bh, wq, wk)
    check(sel(bx), want, torch.float32, f"dimwise fp32 B{B} (tiled {tiled})")
    assert fpscan_amd.lookback_overruns() == before
