"""Seeded random configurations across every entry point and path, against the float64 oracle.

Each case draws its own shape, dtype, gate range and path from a generator seeded by the case
number, so a failure names a case that reruns identically:
* row scans through the torch API: automatic, streamed or tiled (`set_tiling`), and streamed
  with forced launch shapes (`set_launch_override`: waves per row, ring depth), forward,
  reverse and the fused backward;
* row scans through the C ABI on padded strides (the padding must come back untouched);
* channel-last scans (any seqlen, dim a multiple of the 16-byte vector), every path;
* the fused softplus gates, forward, reverse and backward (grad_z, grad_rate, grad_tokens);
* dimwise_forward at any supported seqlen on the automatic, row and tiled paths, on keys
  spaced so that the first-maximum selection is unambiguous in every dtype.
The bar is the tests' normwise one (north star: 1e-5 fp32, 5e-3 fp16, 2e-2 bf16); grad_rate,
a sum over batch and seqlen per dim, gets max(bar, 1e-4) as in test_softplus_gpu.py.
"""
import ctypes
import os
import random

import numpy as np
import pytest
import torch

import fpscan_amd
import oracle
from fpscan_amd import ops
from scan_helpers import DEVICE, DTYPES, NORM_TOL

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]

CASES = 108
MAX_ELEMENTS = 1 << 22
CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _lib():
    lib = ctypes.CDLL(os.path.join(os.path.dirname(fpscan_amd.__file__), "libfpscan_hip.so"))
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.fpscan_scan_fwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i32, i32, vp,
                                    ctypes.c_size_t, vp]
    lib.fpscan_scan_bwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, vp,
                                    ctypes.c_size_t, vp]
    lib.fpscan_workspace_bytes.argtypes = [i64, i64, i64, i32, i32]
    lib.fpscan_workspace_bytes.restype = ctypes.c_size_t
    return lib


class paths:
    """Path selection and launch shape for the duration of one case."""

    def __init__(self, tiling=0, waves=0, ring=0):
        self.tiling, self.waves, self.ring = tiling, waves, ring

    def __enter__(self):
        ops.set_tiling(self.tiling)
        ops.set_launch_override(self.waves, self.ring)

    def __exit__(self, *exc):
        ops.set_tiling(0)
        ops.set_launch_override(0, 0)


def _gates_tokens(rng, gen, shape, dtype, axis_len):
    lo = rng.choice([0.0, 0.5, 0.9, 0.99])
    gates = lo + (1.0 - lo) * torch.rand(shape, generator=gen)
    tokens = torch.randn(shape, generator=gen)
    if rng.random() < 0.5:
        tokens = tokens / axis_len
    return gates.to(dtype), tokens.to(dtype)


def _row_shape(rng):
    L = 2 ** rng.randint(5, 16)
    rows = rng.randint(1, min(max(1, MAX_ELEMENTS // L), 4096))
    B = rng.randint(1, 4)
    return B, max(1, rows // B), L


def _assert_within(errs, dtype, desc):
    bad = {k: v for k, v in errs.items() if not v <= NORM_TOL[dtype]}
    assert not bad, f"{desc}: normwise errors above {NORM_TOL[dtype]}: {bad}"


def _rows_api(rng, gen, dtype):
    B, D, L = _row_shape(rng)
    tiling = rng.choice([0, 1, 2, 2])
    waves = ring = 0
    if tiling == 1 and rng.random() < 0.5:
        waves, ring = rng.choice([1, 2, 4, 8, 16]), rng.choice([1, 2, 3, 4])
    desc = f"rows ({B}, {D}, {L}) {dtype} tiling {tiling} launch ({waves}, {ring})"
    g, x = _gates_tokens(rng, gen, (B, D, L), dtype, L)
    go = torch.randn((B, D, L), generator=gen).to(dtype)
    with paths(tiling, waves, ring):
        gd, xd = g.to(DEVICE), x.to(DEVICE)
        y = fpscan_amd.scan_forward(gd, xd)
        yr = fpscan_amd.scan_forward(gd, xd, reverse=True)
        gg, gx = fpscan_amd.scan_backward(gd, y, go.to(DEVICE))
        torch.cuda.synchronize()
    y = y.cpu()
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, y, go)
    _assert_within({"forward": oracle.normwise_error(y, oracle.scan_f64(g, x)),
                    "reverse": oracle.normwise_error(yr, oracle.scan_f64(g, x, True)),
                    "grad_tokens": oracle.normwise_error(gx, gx_ref),
                    "grad_gates": oracle.normwise_error(gg, gg_ref)}, dtype, desc)


def _rows_abi_strided(rng, gen, dtype):
    B, D, L = _row_shape(rng)
    tiled = rng.random() < 0.5
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    sd = L + vec * rng.randint(0, 8)
    sb = D * sd + vec * rng.randint(0, 8)
    reverse = rng.random() < 0.3
    desc = f"C ABI ({B}, {D}, {L}) strides ({sb}, {sd}) {dtype} tiled {tiled} reverse {reverse}"
    g, x = _gates_tokens(rng, gen, (B, D, L), dtype, L)
    go = torch.randn((B, D, L), generator=gen).to(dtype)

    def embed(t, fill):
        buf = torch.full((B * sb,), fill, dtype=dtype)
        buf.as_strided((B, D, L), (sb, sd, 1)).copy_(t)
        return buf.to(DEVICE)

    def view(buf):
        return buf.cpu().as_strided((B, D, L), (sb, sd, 1))

    lib = _lib()
    code, stream = CODE[dtype], torch.cuda.current_stream().cuda_stream
    gb, xb, gob = embed(g, 7.0), embed(x, 7.0), embed(go, 7.0)
    yb, revb, ggb, gxb = (embed(torch.zeros_like(x), -3.0) for _ in range(4))

    def workspace(op):
        n = lib.fpscan_workspace_bytes(B, D, L, code, op) if tiled else 0
        return n, torch.full((max(n, 8),), 0xA5, dtype=torch.uint8, device=DEVICE)

    with paths(2 if tiled else 1):
        n, ws = workspace(0)
        for out, rev in ((yb, 0), (revb, 1)):
            assert lib.fpscan_scan_fwd(gb.data_ptr(), xb.data_ptr(), out.data_ptr(), B, D, L, sb,
                                       sd, code, rev, ws.data_ptr() if n else None, n,
                                       stream) == 0
        n, ws = workspace(1)
        assert lib.fpscan_scan_bwd(gb.data_ptr(), yb.data_ptr(), gob.data_ptr(), ggb.data_ptr(),
                                   gxb.data_ptr(), B, D, L, sb, sd, code,
                                   ws.data_ptr() if n else None, n, stream) == 0
        torch.cuda.synchronize()
    y = view(yb)
    gg_ref, gx_ref = oracle.scan_bwd_f64(g, y, go)
    _assert_within({"forward": oracle.normwise_error(y, oracle.scan_f64(g, x)),
                    "reverse": oracle.normwise_error(view(revb), oracle.scan_f64(g, x, True)),
                    "grad_tokens": oracle.normwise_error(view(gxb), gx_ref),
                    "grad_gates": oracle.normwise_error(view(ggb), gg_ref)}, dtype, desc)
    pad = torch.ones(B * sb, dtype=torch.bool)
    pad.as_strided((B, D, L), (sb, sd, 1)).fill_(False)
    for buf in (yb, revb, ggb, gxb):
        assert bool((buf.cpu()[pad] == -3.0).all()), f"{desc}: padding was written"


def _channel_last(rng, gen, dtype):
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    D = vec * rng.randint(1, 128)
    L = rng.randint(1, 70000) if rng.random() < 0.7 else 2 ** rng.randint(0, 16)
    B = rng.randint(1, 8)
    while B * L * D > MAX_ELEMENTS:
        L = max(1, L // 2)
    tiling = rng.choice([0, 1, 2, 2])
    desc = f"channel-last ({B}, {L}, {D}) {dtype} tiling {tiling}"
    g, x = _gates_tokens(rng, gen, (B, L, D), dtype, L)
    go = torch.randn((B, L, D), generator=gen).to(dtype)
    with paths(tiling):
        gd, xd = g.to(DEVICE), x.to(DEVICE)
        y = fpscan_amd.scan_forward_channel_last(gd, xd)
        yr = fpscan_amd.scan_forward_channel_last(gd, xd, reverse=True)
        gg, gx = fpscan_amd.scan_backward_channel_last(gd, y, go.to(DEVICE))
        torch.cuda.synchronize()
    y = y.cpu()
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, y, go)
    _assert_within({"forward": oracle.normwise_error(y, oracle.scan_f64_channel_last(g, x)),
                    "reverse": oracle.normwise_error(yr,
                                                     oracle.scan_f64_channel_last(g, x, True)),
                    "grad_tokens": oracle.normwise_error(gx, gx_ref),
                    "grad_gates": oracle.normwise_error(gg, gg_ref)}, dtype, desc)


def _softplus(rng, gen, dtype):
    B, D, L = _row_shape(rng)
    z_mean = rng.choice([-9.0, -3.0, 0.0, 3.0])
    desc = f"softplus ({B}, {D}, {L}) {dtype} z ~ N({z_mean}, 2)"
    z = (z_mean + 2.0 * torch.randn((B, D, L), generator=gen)).to(dtype)
    # rates that keep the gates decaying (about 0.99 per step where z is below 0): a long
    # undecayed sum carries its own fp32 accumulation error close to the fp32 bar
    scale = 0.01 * float(np.exp(-z_mean)) if z_mean < 0 else 0.05
    rate = (scale * (0.5 + 1.5 * torch.rand(D, generator=gen))).float()
    x = (torch.randn((B, D, L), generator=gen) / L).to(dtype)
    go = torch.randn((B, D, L), generator=gen).to(dtype)
    zd, rd, xd = z.to(DEVICE), rate.to(DEVICE), x.to(DEVICE)
    y = fpscan_amd.scan_forward_softplus(zd, rd, xd)
    yr = fpscan_amd.scan_forward_softplus(zd, rd, xd, reverse=True)
    gz, gr, gx = fpscan_amd.scan_backward_softplus(zd, rd, y, go.to(DEVICE))
    torch.cuda.synchronize()
    y = y.cpu()
    gz_ref, gr_ref, gx_ref = oracle.scan_bwd_softplus_f64(z, rate, y, go)
    _assert_within({"forward": oracle.normwise_error(y, oracle.scan_softplus_f64(z, rate, x)),
                    "reverse": oracle.normwise_error(yr,
                                                     oracle.scan_softplus_f64(z, rate, x, True)),
                    "grad_tokens": oracle.normwise_error(gx, gx_ref),
                    "grad_z": oracle.normwise_error(gz, gz_ref)}, dtype, desc)
    err = oracle.normwise_error(gr, gr_ref)
    assert err <= max(NORM_TOL[dtype], 1e-4), f"{desc}: grad_rate normwise error {err:.3e}"


def _dimwise(rng, gen, dtype):
    seqlens = sorted(oracle.DIMWISE_GEOMETRY)
    L = rng.choice(seqlens + [s for s in seqlens if s >= 8192])  # the tiled seqlens twice
    B, D = rng.randint(1, 3), rng.randint(1, 24)
    tiling = rng.choice([0, 1, 2, 2])
    sign = rng.choice([1.0, -1.0])
    desc = f"dimwise ({B}, {D}, {L}) {dtype} tiling {tiling} sign {sign}"
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    ax = 0.99 + 0.01 * torch.rand(B, D, L, generator=gen)
    bx = sign * (0.5 + 0.5 * torch.rand(B, D, L, generator=gen)) / P
    ranks = torch.rand(B, D, W, generator=gen).argsort(dim=-1).argsort(dim=-1).double()
    bh = torch.randn(B, D, W * C, generator=gen) / (W * C)
    bh[:, :, :W] = ((-1.0 + 2.0 * ranks / max(W - 1, 1)) / 4).float()
    wq = 0.01 * torch.rand(D, generator=gen)
    wk = 0.01 * torch.rand(D, generator=gen)
    t = [v.to(dtype).contiguous() for v in (ax, bx, bh, wq, wk)]
    want = oracle.dimwise_f64(*t)
    dev = [v.to(DEVICE) for v in t]
    with paths(tiling):
        fpscan_amd.dimwise_forward(*dev)
        torch.cuda.synchronize()
    _assert_within({"dimwise": oracle.normwise_error(dev[1].cpu(), want)}, dtype, desc)


KINDS = [_rows_api, _rows_api, _rows_abi_strided, _channel_last, _softplus, _dimwise]


@pytest.mark.parametrize("case", range(CASES))
def test_random_configuration_matches_oracle(case):
    rng = random.Random(9001 + case)
    gen = torch.Generator().manual_seed(77 + case)
    kind = KINDS[case % len(KINDS)]
    dtype = DTYPES[rng.randrange(len(DTYPES))]
    kind(rng, gen, dtype)
    assert fpscan_amd.lookback_overruns() == 0
