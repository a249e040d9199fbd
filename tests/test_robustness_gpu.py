"""GPU tests of the failure and aliasing contracts around the tiled paths.

* In-place use: ``out`` may alias ``tokens`` or ``gates`` (include/fpscan_hip.h; the
  reference's caller contract is fpscan/ops.py:55-57), on the streaming and the tiled row path
  and at the size where tiling is the automatic choice.
* Look-back waits that give up: a test hook keeps one tile from ever publishing its map and
  lowers the poll bound, so the waits on it give up while every kernel still exits normally.
  The affected tiles must come out NaN (never plausible numbers), every other value must equal
  an unhooked run bit for bit, and the per-device counter must report the given-up waits. The
  reference has no cross-workgroup wait (full_scan.cu:77-175 keeps every carry in one block).
* Long runs: hundreds of back-to-back tiled calls (row and channel-last kernels) at the
  headline size and the one-GPU share, outputs filled with NaN before each call, so that a tile
  that is dropped or a wait that gives up in one call in a hundred is seen; the tiled dimwise
  kernel in place, its input restored before each call and every output equal to the first.
* HIP graph capture through the torch binding is refused with a RuntimeError before anything
  is launched (the capture is begun and ended with the runtime's own calls, no graph is
  instantiated).
"""
import ctypes

import pytest
import torch

import bench
import fpscan_amd
from fpscan_amd import ops
from scan_helpers import DEVICE, bits_equal, make_inputs

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]


class tiling:
    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        ops.set_tiling(self.mode)

    def __exit__(self, *exc):
        ops.set_tiling(0)


class lookback_hook:
    """Tile `tile` (claim order) never publishes; waits give up after `spin` polls."""

    def __init__(self, tile, spin=64):
        self.tile, self.spin = tile, spin

    def __enter__(self):
        ops.set_lookback_test_hook(self.tile, self.spin)

    def __exit__(self, *exc):
        ops.set_lookback_test_hook(-1, 0)


# ------------------------------------------------------------------ in-place use
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("mode", [1, 2], ids=["stream", "tiled"])
@pytest.mark.parametrize("alias", ["tokens", "gates"])
@pytest.mark.parametrize("reverse", [False, True], ids=["fwd", "rev"])
def test_in_place_equals_out_of_place(dtype, mode, alias, reverse):
    """Rows of 64 (bf16) or 128 (fp32) sub-chunks: 4 or 8 tiles per row when tiled."""
    g, x = make_inputs(4, 8, 32768, dtype, seed=5)
    g, x = g.to(DEVICE), x.to(DEVICE)
    with tiling(mode):
        want = fpscan_amd.scan_forward(g, x, reverse)
        gi, xi = g.clone(), x.clone()
        target = xi if alias == "tokens" else gi
        got = fpscan_amd.scan_forward(gi, xi, reverse, out=target)
        torch.cuda.synchronize()
    assert got.data_ptr() == target.data_ptr()
    assert bits_equal(got, want), f"in place on {alias} differs ({dtype}, mode {mode})"


def test_in_place_at_the_automatic_tiling_size():
    """bf16 (4, 1024, 65536): 512 MiB per tensor, tiled by default."""
    B, D, L = 4, 1024, 65536
    assert ops._load_extension().workspace_bytes(B, D, L, 2, 0) > 0  # the tiled path
    g, x, _ = bench.make_inputs(B, D, L, torch.bfloat16, "mamba", seed=9, grad=False)
    want = fpscan_amd.scan_forward(g, x)
    for alias in ("tokens", "gates"):
        gi, xi = g.clone(), x.clone()
        target = xi if alias == "tokens" else gi
        fpscan_amd.scan_forward(gi, xi, out=target)
        torch.cuda.synchronize()
        assert bits_equal(target, want), f"in place on {alias} differs"
        del gi, xi, target


def test_partial_overlaps_are_refused_before_any_launch():
    """An output may be one of its inputs exactly (forward scans) but never part of one, and
    backward outputs share no byte with inputs or each other: a lane would overwrite elements
    another lane still reads (the backward reads gates[t+1] and out[t-1] across lanes)."""
    shape, n = (2, 4, 64), 2 * 4 * 64
    buf = torch.randn(n + 64, device=DEVICE)
    a, shifted = buf[:n].view(shape), buf[64:n + 64].view(shape)  # overlap by 7 of 8 rows
    x = torch.randn(shape, device=DEVICE)
    keep = buf.clone()
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.scan_forward(a, x, out=shifted)
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.scan_forward(x, a, out=shifted)
    y = fpscan_amd.scan_forward(x, x.clone())
    go = torch.randn_like(y)
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.scan_backward(a, y, go, grad_gates=shifted, grad_tokens=torch.empty_like(y))
    with pytest.raises(RuntimeError, match="overlap"):
        fpscan_amd.scan_backward(x, y, go, grad_gates=a, grad_tokens=shifted)
    # channel-last (batch, seqlen, dim) and the fused gates
    cl = (2, 8, 32)
    a_cl, s_cl = buf[:n].view(cl), buf[64:n + 64].view(cl)
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.scan_forward_channel_last(a_cl, torch.randn(cl, device=DEVICE), out=s_cl)
    with pytest.raises(RuntimeError, match="overlap"):
        fpscan_amd.scan_backward_channel_last(x.view(cl), y.view(cl), go.view(cl),
                                              grad_gates=a_cl, grad_tokens=s_cl)
    rate = torch.ones(4, device=DEVICE)
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.scan_forward_softplus(a, rate, x, out=shifted)
    torch.cuda.synchronize()
    assert torch.equal(buf, keep), "a refused call wrote into its outputs"
    # exact aliasing stays allowed
    want = fpscan_amd.scan_forward(a.clone(), x)
    fpscan_amd.scan_forward(a, x, out=a)
    assert bits_equal(a, want)


# ------------------------------------------------------------------ look-back waits that give up
def _tile_span(seg, tile_len, L, reverse):
    """Element range [lo, hi) of tile `seg` of a row, in memory order."""
    if reverse:
        return L - (seg + 1) * tile_len, L - seg * tile_len
    return seg * tile_len, (seg + 1) * tile_len


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("op", ["fwd", "rev", "bwd"])
def test_row_overrun_poisons_and_is_counted(dtype, op):
    """3 rows of 4 tiles; tile 1 (row 0, second tile in processing order) never publishes, so
    tiles 2 and 3 of row 0 give up waiting: exactly their elements are NaN, the rest equals an
    unhooked run, and the device counter grows by the waits that gave up."""
    tile_len = 8192 if dtype == torch.bfloat16 else 4096  # 16 sub-chunks
    L = 4 * tile_len
    g, x = make_inputs(1, 3, L, dtype, seed=11)
    go = torch.randn(g.shape, generator=torch.Generator().manual_seed(12)).to(dtype)
    g, x, go = g.to(DEVICE), x.to(DEVICE), go.to(DEVICE)

    with tiling(2):
        y = fpscan_amd.scan_forward(g, x)  # the backward's saved output, from an unhooked run

        def run():
            if op == "bwd":
                return list(fpscan_amd.scan_backward(g, y, go))
            return [fpscan_amd.scan_forward(g, x, op == "rev")]

        want = run()
        before = fpscan_amd.lookback_overruns()
        with lookback_hook(1):
            got = run()
        torch.cuda.synchronize()
        after = fpscan_amd.lookback_overruns()
    assert after - before >= 2, f"given-up waits not counted ({before} -> {after})"
    lo, hi = _tile_span(2, tile_len, L, op != "fwd")
    lo3, hi3 = _tile_span(3, tile_len, L, op != "fwd")
    poisoned = torch.zeros(g.shape, dtype=torch.bool)
    poisoned[0, 0, min(lo, lo3):max(hi, hi3)] = True
    for a, b in zip(got, want):
        a, b = a.cpu(), b.cpu()
        assert torch.isnan(a[poisoned]).all(), "a tile whose wait gave up must be NaN"
        assert bits_equal(a[~poisoned], b[~poisoned]), "tiles that waited normally changed"
    with pytest.raises(RuntimeError, match="gave up"):
        fpscan_amd.check_lookback()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("op", ["fwd", "rev", "bwd"])
def test_channel_last_overrun_poisons_and_is_counted(dtype, op):
    """One chain (batch 1, 64 columns) of 16 tiles, so the wide look-back (few chains): the
    carry into tile k composes the aggregates of tiles k-1 .. k-15 (back to the chain start)
    onto the end value of tile k-16. Tile 1 never publishes its aggregates, so tiles 2..15
    give up waiting and must be NaN (the narrow depth 5 makes that tiles 2..6; the test holds
    either way); tiles 0 and 1 must equal an unhooked run. Once one wait of a launch has given
    up, the others give up at once, so which later tiles are also NaN depends on timing -- but
    none may hold a value that is neither NaN nor the unhooked one."""
    steps = 128 if dtype == torch.bfloat16 else 64
    L = 16 * steps
    gen = torch.Generator().manual_seed(21)
    g = (0.9 + 0.1 * torch.rand(1, L, 64, generator=gen)).to(dtype).to(DEVICE)
    x = torch.randn(1, L, 64, generator=gen).to(dtype).to(DEVICE)
    go = torch.randn(1, L, 64, generator=gen).to(dtype).to(DEVICE)

    with tiling(2):
        y = fpscan_amd.scan_forward_channel_last(g, x)

        def run():
            if op == "bwd":
                return list(fpscan_amd.scan_backward_channel_last(g, y, go))
            return [fpscan_amd.scan_forward_channel_last(g, x, op == "rev")]

        want = run()
        before = fpscan_amd.lookback_overruns()
        with lookback_hook(1):
            got = run()
        torch.cuda.synchronize()
        after = fpscan_amd.lookback_overruns()
    assert after > before, f"given-up waits not counted ({before} -> {after})"

    def steps_of(k0, k1):  # time steps of tiles k0 .. k1-1 in processing order
        if op == "fwd":
            return slice(k0 * steps, k1 * steps)
        return slice(L - k1 * steps, L - k0 * steps)

    for a, b in zip(got, want):
        a, b = a.cpu(), b.cpu()
        assert bits_equal(a[:, steps_of(0, 2)], b[:, steps_of(0, 2)]), "tiles 0, 1 changed"
        assert torch.isnan(a[:, steps_of(2, 7)]).all(), "tiles 2..6 must be NaN"
        nan = torch.isnan(a)
        assert bits_equal(a[~nan], b[~nan]), "a value is neither NaN nor the unhooked one"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("op", ["fwd", "rev", "bwd"])
def test_channel_last_narrow_overrun_poisons_and_is_counted(dtype, op):
    """48 chains (64 columns each) of 16 tiles, so the narrow look-back (depth 5; the wide
    one is for fewer chains). Tile 1 in claim order, the first tile of chain 1, never
    publishes its aggregate: tiles 1..5 of that chain give up waiting and must be NaN, as must
    every later tile whose carry starts from one of their end values (tiles 7..11, 13..15);
    tiles 6 and 12 start from the end values of tiles 0 and 6 and may come out right. Chain
    1's first tile must equal an unhooked run; every other value is NaN (a wait of the launch
    gave up after the overrun) or equal to the unhooked run, never anything else."""
    steps = 128 if dtype == torch.bfloat16 else 64
    L, D = 16 * steps, 48 * 64
    gen = torch.Generator().manual_seed(23)
    g = (0.9 + 0.1 * torch.rand(1, L, D, generator=gen)).to(dtype).to(DEVICE)
    x = torch.randn(1, L, D, generator=gen).to(dtype).to(DEVICE)
    go = torch.randn(1, L, D, generator=gen).to(dtype).to(DEVICE)

    with tiling(2):
        y = fpscan_amd.scan_forward_channel_last(g, x)

        def run():
            if op == "bwd":
                return list(fpscan_amd.scan_backward_channel_last(g, y, go))
            return [fpscan_amd.scan_forward_channel_last(g, x, op == "rev")]

        want = run()
        before = fpscan_amd.lookback_overruns()
        with lookback_hook(1):
            got = run()
        torch.cuda.synchronize()
        after = fpscan_amd.lookback_overruns()
    assert after > before, f"given-up waits not counted ({before} -> {after})"

    def steps_of(k0, k1):  # time steps of tiles k0 .. k1-1 in processing order
        if op == "fwd":
            return slice(k0 * steps, k1 * steps)
        return slice(L - k1 * steps, L - k0 * steps)

    chain1 = slice(64, 128)
    for a, b in zip(got, want):
        a, b = a.cpu(), b.cpu()
        assert bits_equal(a[:, steps_of(0, 1), chain1], b[:, steps_of(0, 1), chain1]), \
            "chain 1's first tile changed"
        for k0, k1 in ((1, 6), (7, 12), (13, 16)):
            assert torch.isnan(a[:, steps_of(k0, k1), chain1]).all(), \
                f"chain 1's tiles {k0}..{k1 - 1} must be NaN"
        nan = torch.isnan(a)
        assert bits_equal(a[~nan], b[~nan]), "a value is neither NaN nor the unhooked one"


def test_hook_off_restores_normal_runs():
    """After the hook is cleared the tiled path publishes and waits normally again."""
    g, x = make_inputs(1, 3, 32768, torch.bfloat16, seed=13)
    g, x = g.to(DEVICE), x.to(DEVICE)
    with tiling(2):
        with lookback_hook(1):
            fpscan_amd.scan_forward(g, x)
        torch.cuda.synchronize()
        before = fpscan_amd.lookback_overruns()
        y = fpscan_amd.scan_forward(g, x)
        torch.cuda.synchronize()
        assert fpscan_amd.lookback_overruns() == before
    assert not torch.isnan(y).any()


# ------------------------------------------------------------------ no tile is ever dropped
@pytest.mark.parametrize("dtype,op,calls", [(torch.float32, "fwd", 400),
                                            (torch.bfloat16, "fwd", 200),
                                            (torch.float32, "rev", 200),
                                            (torch.float32, "bwd", 100),
                                            (torch.bfloat16, "bwd", 100)],
                         ids=["f32-fwd", "bf16-fwd", "f32-rev", "f32-bwd", "bf16-bwd"])
def test_repeated_headline_calls_drop_no_tile(dtype, op, calls):
    """Hundreds of back-to-back tiled calls (forward, reverse, backward) at the headline shape
    (8, 1024, 65536): outputs filled with NaN before each call come back finite every time, no
    wait gives up, and the last call equals the first bit for bit. A workgroup that left its loop on an empty ring
    while claims were still in flight dropped the tiles those claims held (their outputs were
    never written and the later tiles of their rows gave up waiting), a few calls in a
    hundred; the loop now ends only on the claim stream's end."""
    g, x, go = bench.make_inputs(8, 1024, 65536, dtype, "mamba", seed=21)
    y = fpscan_amd.scan_forward(g, x)
    outs = [torch.empty_like(x)] if op != "bwd" else [torch.empty_like(x), torch.empty_like(x)]
    nan_seen = torch.zeros((), dtype=torch.bool, device=DEVICE)
    first = None
    torch.cuda.synchronize()
    before = fpscan_amd.lookback_overruns()
    for i in range(calls):
        for o in outs:
            o.fill_(float("nan"))
        if op != "bwd":
            fpscan_amd.scan_forward(g, x, op == "rev", outs[0])
        else:
            fpscan_amd.scan_backward(g, y, go, outs[0], outs[1])
        for o in outs:
            nan_seen |= torch.isnan(o).any()
        if i == 0:
            first = [o.clone() for o in outs]
    torch.cuda.synchronize()
    after = fpscan_amd.lookback_overruns()
    assert after == before, f"{after - before} look-back waits gave up in {calls} calls"
    assert not bool(nan_seen), "an output element was left unwritten or poisoned"
    for a, b in zip(outs, first):
        assert torch.equal(a.view(torch.int16 if a.element_size() == 2 else torch.int32),
                           b.view(torch.int16 if b.element_size() == 2 else torch.int32))


@pytest.mark.parametrize("batch,op,calls", [(8, "fwd", 100), (1, "fwd", 200), (1, "bwd", 200)],
                         ids=["b8-fwd", "b1-fwd", "b1-bwd"])
def test_repeated_channel_last_tiled_calls_drop_no_tile(batch, op, calls):
    """The channel-last tiled kernel (its own look-back across workgroups) under the same
    long-run check: (batch, 65536, 1024) bf16, outputs filled with NaN before each call, every
    output written, no wait given up, the last call equal to the first bit for bit."""
    g, x, go = bench.make_inputs(batch, 65536, 1024, torch.bfloat16, "mamba", seed=22)
    y = fpscan_amd.scan_forward_channel_last(g, x)
    outs = [torch.empty_like(x)] if op == "fwd" else [torch.empty_like(x), torch.empty_like(x)]
    nan_seen = torch.zeros((), dtype=torch.bool, device=DEVICE)
    first = None
    torch.cuda.synchronize()
    before = fpscan_amd.lookback_overruns()
    for i in range(calls):
        for o in outs:
            o.fill_(float("nan"))
        if op == "fwd":
            fpscan_amd.scan_forward_channel_last(g, x, False, outs[0])
        else:
            fpscan_amd.scan_backward_channel_last(g, y, go, outs[0], outs[1])
        for o in outs:
            nan_seen |= torch.isnan(o).any()
        if i == 0:
            first = [o.clone() for o in outs]
    torch.cuda.synchronize()
    after = fpscan_amd.lookback_overruns()
    assert after == before, f"{after - before} look-back waits gave up in {calls} calls"
    assert not bool(nan_seen), "an output element was left unwritten or poisoned"
    for a, b in zip(outs, first):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("dtype,calls", [(torch.bfloat16, 200), (torch.float32, 100)],
                         ids=["bf16", "f32"])
def test_repeated_dimwise_tiled_calls_drop_no_tile(dtype, calls):
    """dimwise_forward's tiled path at (8, 1024, 65536), in place: Bx is restored from the same
    input before each call, and every call's output must equal the first bit for bit (a tile
    left unwritten keeps its input, a wait that gave up leaves NaN) with no wait given up."""
    B, D, L = 8, 1024, 65536
    assert ops.dimwise_workspace_bytes(B, D, L, dtype) > 0, "the tiled path is the default here"
    G = fpscan_amd.dimwise_groups(L)
    gen = torch.Generator(device=DEVICE).manual_seed(23)
    ax = (0.99 + 0.01 * torch.rand(B, D, L, generator=gen, device=DEVICE)).to(dtype)
    bx0 = (torch.randn(B, D, L, generator=gen, device=DEVICE) / G).to(dtype)
    bh = (torch.randn(B, D, G, generator=gen, device=DEVICE) / G).to(dtype)
    wq = (0.01 * torch.rand(D, generator=gen, device=DEVICE)).to(dtype)
    wk = (0.01 * torch.rand(D, generator=gen, device=DEVICE)).to(dtype)
    bits = torch.int16 if dtype != torch.float32 else torch.int32
    bx = torch.empty_like(bx0)
    differs = torch.zeros((), dtype=torch.bool, device=DEVICE)
    first = None
    torch.cuda.synchronize()
    before = fpscan_amd.lookback_overruns()
    for i in range(calls):
        bx.copy_(bx0)
        fpscan_amd.dimwise_forward(ax, bx, bh, wq, wk)
        if i == 0:
            first = bx.clone()
        else:
            differs |= (bx.view(bits) != first.view(bits)).any()
    torch.cuda.synchronize()
    after = fpscan_amd.lookback_overruns()
    assert after == before, f"{after - before} look-back waits gave up in {calls} calls"
    assert not bool(differs), "a call's output differs from the first call's"
    assert not torch.isnan(first).any()
    assert not torch.equal(first.view(bits), bx0.view(bits))


# ------------------------------------------------------------------ graph capture is refused
def test_graph_capture_is_refused_before_any_launch():
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch has loaded (same SONAME)
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    g, x = make_inputs(2, 4, 1024, torch.bfloat16, seed=14)
    g, x = g.to(DEVICE), x.to(DEVICE)
    out = torch.empty_like(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        relaxed = 2  # hipStreamCaptureModeRelaxed
        assert hip.hipStreamBeginCapture(side.cuda_stream, relaxed) == 0
        graph = ctypes.c_void_p()
        try:
            with pytest.raises(RuntimeError, match="graph capture"):
                fpscan_amd.scan_forward(g, x, out=out)
        finally:
            assert hip.hipStreamEndCapture(side.cuda_stream, ctypes.byref(graph)) == 0
            if graph.value:
                hip.hipGraphDestroy(graph)
    torch.cuda.synchronize()
    # eager use on the same stream afterwards is unaffected
    with torch.cuda.stream(side):
        y = fpscan_amd.scan_forward(g, x)
    torch.cuda.synchronize()
    assert bits_equal(y, fpscan_amd.scan_forward(g, x))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_dimwise_overrun_poisons_and_is_counted(dtype):
    """dimwise_forward's tiled path: 3 rows of 4 tiles; tile 1 (row 0, second tile) never
    publishes its map, so tiles 2 and 3 of row 0 give up waiting. Their carry is NaN: group 0
    of each of their chunks (which continues from the carry) must be NaN, every other element
    of them NaN or equal to an unhooked run (a group whose r does not go through group 0 is
    independent of the carry), and everything outside them equal to the unhooked run; the
    device counter grows by the waits that gave up."""
    tile_len = 8192 if dtype == torch.bfloat16 else 4096  # 16 KiB
    L = 4 * tile_len
    gen = torch.Generator().manual_seed(13)
    G = fpscan_amd.dimwise_groups(L)
    ax = 0.99 + 0.01 * torch.rand(1, 3, L, generator=gen)
    bx = torch.randn(1, 3, L, generator=gen) / G
    bh = torch.randn(1, 3, G, generator=gen) / G
    wq, wk = 0.01 * torch.rand(3, generator=gen), 0.01 * torch.rand(3, generator=gen)
    t = [v.to(dtype).to(DEVICE) for v in (ax, bx, bh, wq, wk)]
    with tiling(2):
        want = t[1].clone()
        fpscan_amd.dimwise_forward(t[0], want, *t[2:])
        before = fpscan_amd.lookback_overruns()
        with lookback_hook(1):
            got = t[1].clone()
            fpscan_amd.dimwise_forward(t[0], got, *t[2:])
            torch.cuda.synchronize()
        after = fpscan_amd.lookback_overruns()
    assert after - before >= 2, f"given-up waits not counted ({before} -> {after})"
    got, want = got.cpu(), want.cpu()
    hit = torch.zeros(got.shape, dtype=torch.bool)
    hit[0, 0, 2 * tile_len:] = True
    assert torch.equal(got[~hit], want[~hit]), "tiles that waited normally changed"
    g, w = got[0, 0, 2 * tile_len:], want[0, 0, 2 * tile_len:]
    assert (torch.isnan(g) | (g == w)).all(), "a value that is neither NaN nor the unhooked one"
    group0 = g.view(-1, 4096)[:, :128]
    assert torch.isnan(group0).all(), "group 0 of a tile whose wait gave up must be NaN"
    with pytest.raises(RuntimeError, match="gave up"):
        fpscan_amd.check_lookback()
