"""GPU parity tests of the tiled channel-last scan: one pass over (batch, seqlen, dim) tensors
with a look-back along seqlen (chains of 64 columns, tiles of 128 steps in 2-byte types and 64
in fp32), against the CPU oracle (oracle.scan_f64_channel_last / scan_bwd_f64_channel_last,
pinned by tests/test_oracle.py).

fpscan_set_tiling(2) forces the tiled path on most shapes here; the automatic choice takes it
wherever there are too few strips for one pass, or a tensor is 512 MiB or more, and seqlen
spans more than one tile (tested at its real size last). Besides the oracle: the
workspace after a call (every tile's aggregate published, no wait overrun, claim counters at
or past their group sizes), bit-exactness on integer data, run-to-run determinism and the
reverse = flip(forward(flip)) identity bit for bit (the carry into a tile is always composed
the same way, whatever the timing), agreement with the one-pass and segmented paths, padded
strides and autograd.
"""
import ctypes
import os

import pytest
import torch

import fpscan_amd
import oracle
from scan_helpers import DEVICE, DTYPES, NORM_TOL, bits_equal, check

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]

_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_EXTRA_WORDS = 16 * (1 + 8)  # overrun word, then 8 claim counters 16 words apart


def cl_inputs(batch, seqlen, dim, dtype, seed=0):
    """test_fpscan.py:25-29 distributions in (batch, seqlen, dim) layout."""
    gen = torch.Generator().manual_seed(seed)
    gates = 0.99 + 0.01 * torch.rand(batch, seqlen, dim, generator=gen)
    tokens = torch.randn(batch, seqlen, dim, generator=gen) / max(seqlen, 1)
    return gates.to(dtype).contiguous(), tokens.to(dtype).contiguous()


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(os.path.join(os.path.dirname(fpscan_amd.__file__), "libfpscan_hip.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_scan_fwd_cl.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                       ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fpscan_scan_bwd_cl.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                       vp, ctypes.c_size_t, vp]
    lib.fpscan_workspace_bytes_cl.argtypes = [i64, i64, i64, i64, ctypes.c_int, ctypes.c_int]
    lib.fpscan_workspace_bytes_cl.restype = ctypes.c_size_t
    lib.fpscan_set_tiling.argtypes = [ctypes.c_int]
    return lib


@pytest.fixture
def tiled(lib):
    assert lib.fpscan_set_tiling(2) == 0
    yield
    lib.fpscan_set_tiling(0)


def tile_geometry(batch, seqlen, dim, dtype):
    steps = 16 * (16 // torch.empty((), dtype=dtype).element_size())
    chains = batch * -(-dim // 64)
    nseg = -(-seqlen // steps)
    return chains, nseg, chains * nseg


def check_workspace(ws, batch, seqlen, dim, dtype, what):
    """Every tile published its 64 aggregates, no wait ran into its bound, and each claim
    group's counter reached (at least) its number of tiles."""
    chains, nseg, ntiles = tile_geometry(batch, seqlen, dim, dtype)
    nagg = ntiles * 64
    words = ws[: (nagg * 3 // 2 + _EXTRA_WORDS) * 8].cpu().view(torch.int64)
    aggs = words[:nagg]
    assert (aggs != -1).all(), f"{what}: {(aggs == -1).sum().item()} aggregates unpublished"
    extra = words[nagg * 3 // 2:]
    assert extra[0].item() == 0, f"{what}: {extra[0].item()} look-back waits overran"
    for g in range(8):
        lo, hi = g * chains // 8, (g + 1) * chains // 8
        claimed = extra[16 * (1 + g)].item() & 0xFFFFFFFF
        assert claimed >= (hi - lo) * nseg, f"{what}: group {g} claimed {claimed}"


def abi_fwd(lib, g, x, reverse, ws_check=True):
    B, L, D = x.shape
    out = torch.empty_like(x)
    nbytes = lib.fpscan_workspace_bytes_cl(B, L, D, D, _CODE[x.dtype], 0)
    assert nbytes == tile_geometry(B, L, D, x.dtype)[2] * 768 + _EXTRA_WORDS * 8
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEVICE)
    st = lib.fpscan_scan_fwd_cl(g.data_ptr(), x.data_ptr(), out.data_ptr(), B, L, D, L * D, D,
                                _CODE[x.dtype], int(reverse), ws.data_ptr(), nbytes,
                                torch.cuda.current_stream().cuda_stream)
    assert st == 0
    if ws_check:
        torch.cuda.synchronize()
        check_workspace(ws, B, L, D, x.dtype, f"fwd {tuple(x.shape)} rev={reverse}")
    return out


def abi_bwd(lib, g, y, go):
    B, L, D = g.shape
    gg, gx = torch.empty_like(g), torch.empty_like(g)
    nbytes = lib.fpscan_workspace_bytes_cl(B, L, D, D, _CODE[g.dtype], 1)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEVICE)
    st = lib.fpscan_scan_bwd_cl(g.data_ptr(), y.data_ptr(), go.data_ptr(), gg.data_ptr(),
                                gx.data_ptr(), B, L, D, L * D, D, _CODE[g.dtype], ws.data_ptr(),
                                nbytes, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    check_workspace(ws, B, L, D, g.dtype, f"bwd {tuple(g.shape)}")
    return gg, gx


SHAPES = [
    (1, 1000, 64),    # one chain, ragged last tile
    (3, 700, 200),    # partial strip: 200 = 3 x 64 + 8 columns
    (2, 1, 64),       # one time step
    (4, 129, 64),     # a last tile of one step (2-byte types)
    (2, 4096, 512),   # 16 chains
    (1, 65536, 64),   # one chain of 512 (1024 in fp32) tiles: the deepest dependency chain
    (4, 2048, 1024),  # 64 chains: the narrow look-back of depth 5 in every direction and
                      # type (48-95 chains), consecutive 16-byte pieces of a step per lane
    (8, 2048, 1024),  # 128 chains (look-back depth 3 in the 2-byte forward, else 5; the
                      # 2-byte backward with consecutive lanes on consecutive steps)
]


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_forward_reverse_backward_match_oracle(lib, tiled, dtype, shape):
    g, x = cl_inputs(*shape, dtype, seed=sum(shape))
    go = torch.randn(shape, generator=torch.Generator().manual_seed(5)).to(dtype)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    for rev in (False, True):
        out = abi_fwd(lib, gd, xd, rev)
        check(out, oracle.scan_f64_channel_last(g, x, rev), dtype, f"tiled {shape} rev={rev}")
    y = abi_fwd(lib, gd, xd, False, ws_check=False)
    gg, gx = abi_bwd(lib, gd, y, go.to(DEVICE))
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, y.cpu(), go)
    check(gx, gx_ref, dtype, f"tiled {shape} grad_tokens")
    check(gg, gg_ref, dtype, f"tiled {shape} grad_gates")


# look-back depths: below 48 chains the wide look-back (15 aggregates, one word per wave) in
# every direction and type (8 chains here); 48-95 chains depth 5 everywhere (64 here); 128
# chains 3 in the 2-byte forward and reverse, 5 otherwise; 256 chains 3 in every forward and
# reverse; from 48 chains the backward always 5. Lane orders: the 2-byte backward puts
# consecutive lanes on consecutive steps from 96 chains (128 and 256 here), every other kernel
# on consecutive 16-byte pieces of a step.
DEPTH_SHAPES = [(2, 8192, 256), (4, 1024, 1024), (8, 1024, 1024), (16, 512, 1024)]


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", DEPTH_SHAPES, ids=str)
def test_exact_on_integer_data(lib, tiled, dtype, shape):
    """Gates in {0, 1} and small integer tokens: every partial result is exact, whatever the
    composition order, so the tiled kernels must equal the oracle bit for bit."""
    gen = torch.Generator().manual_seed(21)
    g = (torch.randint(0, 24, shape, generator=gen) > 0).to(dtype)
    x = torch.randint(-3, 4, shape, generator=gen).to(dtype)
    go = torch.randint(-2, 3, shape, generator=gen).to(dtype)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    for rev in (False, True):
        want = torch.from_numpy(oracle.scan_f64_channel_last(g, x, rev))
        if dtype != torch.float32 and want.abs().max() >= 256:
            continue  # not exact in 8-bit mantissas
        assert bits_equal(abi_fwd(lib, gd, xd, rev).cpu(), want.to(dtype)), f"rev={rev}"
    y = oracle.scan_f64_channel_last(g, x, False)
    if dtype == torch.float32 or abs(y).max() < 256:
        yt = torch.from_numpy(y).to(dtype)
        gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, yt, go)
        if dtype == torch.float32 or max(abs(gg_ref).max(), abs(gx_ref).max()) < 256:
            gg, gx = abi_bwd(lib, gd, yt.to(DEVICE), go.to(DEVICE))
            assert bits_equal(gx.cpu(), torch.from_numpy(gx_ref).to(dtype))
            assert bits_equal(gg.cpu(), torch.from_numpy(gg_ref).to(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("batch", [2, 8], ids=["32-chains", "128-chains"])
def test_deterministic_and_reverse_is_mirrored_forward(lib, tiled, dtype, batch):
    """The carry into a tile is composed the same way on every run, so repeated calls agree
    bit for bit, and reverse(g, x) == flip(forward(flip(g), flip(x))) bit for bit (the tiles
    of the reverse pass are the mirrored tiles of the forward pass). Both look-back depths."""
    g, x = cl_inputs(batch, 4000, 1024, dtype, seed=3)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    first = abi_fwd(lib, gd, xd, False, ws_check=False)
    for _ in range(3):
        assert bits_equal(abi_fwd(lib, gd, xd, False, ws_check=False), first)
    rev = abi_fwd(lib, gd, xd, True, ws_check=False)
    mirrored = abi_fwd(lib, gd.flip(1).contiguous(), xd.flip(1).contiguous(), False,
                       ws_check=False).flip(1)
    assert bits_equal(rev, mirrored)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_agrees_with_one_pass_and_segmented_paths(lib, dtype):
    """The three channel-last paths on one problem, each forced through fpscan_set_tiling:
    all within the tolerance of each other and of the oracle."""
    shape = (4, 3000, 320)
    g, x = cl_inputs(*shape, dtype, seed=17)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    want = oracle.scan_f64_channel_last(g, x)
    try:
        assert lib.fpscan_set_tiling(2) == 0
        tiled_out = fpscan_amd.scan_forward_channel_last(gd, xd)
        assert lib.fpscan_set_tiling(1) == 0
        seg_out = fpscan_amd.scan_forward_channel_last(gd, xd)  # 4-8 strips: segments
    finally:
        lib.fpscan_set_tiling(0)
    check(tiled_out, want, dtype, "tiled")
    check(seg_out, want, dtype, "segmented")
    assert oracle.normwise_error(tiled_out, seg_out) <= 2 * NORM_TOL[dtype]


def test_first_gate_nan_does_not_propagate(tiled):
    g, x = cl_inputs(3, 1000, 128, torch.float32, seed=2)
    for rev in (False, True):
        gn = g.clone()
        gn[:, -1 if rev else 0, :] = float("nan")
        out = fpscan_amd.scan_forward_channel_last(gn.to(DEVICE), x.to(DEVICE), reverse=rev)
        assert torch.isfinite(out).all()
        check(out, oracle.scan_f64_channel_last(g, x, rev), torch.float32, f"nan gate rev={rev}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_autograd_matches_oracle(tiled, dtype):
    shape = (2, 3000, 96)
    g, x = cl_inputs(*shape, dtype, seed=13)
    go = torch.randn(shape, generator=torch.Generator().manual_seed(6)).to(dtype)
    gd = g.to(DEVICE).requires_grad_()
    xd = x.to(DEVICE).requires_grad_()
    y = fpscan_amd.pscan_channel_last(gd, xd)
    y.backward(go.to(DEVICE))
    check(y, oracle.scan_f64_channel_last(g, x), dtype, "autograd forward")
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, y.detach().cpu(), go)
    check(xd.grad, gx_ref, dtype, "autograd grad_tokens")
    check(gd.grad, gg_ref, dtype, "autograd grad_gates")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_padded_strides(lib, tiled, dtype):
    """(batch, seqlen, dim) views of a larger buffer: stride_t = dim + pad, stride_b = seqlen *
    stride_t + pad2; results match the oracle and the padding comes back untouched."""
    B, L, D = 3, 2000, 136
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    st = D + 4 * vec
    sb = L * st + 2 * vec
    g, x = cl_inputs(B, L, D, dtype, seed=4)
    go = torch.randn(B, L, D, generator=torch.Generator().manual_seed(2)).to(dtype)

    def embed(t, fill):
        buf = torch.full((B * sb,), fill, dtype=dtype)
        buf.as_strided((B, L, D), (sb, st, 1)).copy_(t)
        return buf.to(DEVICE)

    def view(buf):
        return buf.as_strided((B, L, D), (sb, st, 1))

    gb, xb, gob = embed(g, 7.0), embed(x, 7.0), embed(go, 7.0)
    outb, ggb, gxb = (embed(torch.zeros_like(x), -3.0) for _ in range(3))
    code = _CODE[dtype]
    stream = torch.cuda.current_stream().cuda_stream
    nb = lib.fpscan_workspace_bytes_cl(B, L, D, st, code, 0)
    assert nb == tile_geometry(B, L, D, dtype)[2] * 768 + _EXTRA_WORDS * 8
    ws = torch.empty(nb, dtype=torch.uint8, device=DEVICE)
    assert lib.fpscan_scan_fwd_cl(gb.data_ptr(), xb.data_ptr(), outb.data_ptr(), B, L, D, sb, st,
                                  code, 0, ws.data_ptr(), nb, stream) == 0
    assert lib.fpscan_scan_bwd_cl(gb.data_ptr(), outb.data_ptr(), gob.data_ptr(), ggb.data_ptr(),
                                  gxb.data_ptr(), B, L, D, sb, st, code, ws.data_ptr(), nb,
                                  stream) == 0
    torch.cuda.synchronize()
    out = view(outb).cpu()
    check(out, oracle.scan_f64_channel_last(g, x), dtype, "tiled strided fwd")
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, out, go)
    check(view(gxb).cpu(), gx_ref, dtype, "tiled strided grad_tokens")
    check(view(ggb).cpu(), gg_ref, dtype, "tiled strided grad_gates")
    mask = torch.ones(B * sb, dtype=torch.bool)
    mask.as_strided((B, L, D), (sb, st, 1)).fill_(False)
    for buf in (outb, ggb, gxb):
        assert (buf.cpu()[mask] == -3.0).all(), "padding was written"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_large_problem_with_many_strips_is_tiled(lib, dtype):
    """The automatic choice from 512 MiB per tensor: tiled even with enough strips for one
    pass (bf16 (64, 1024, 8192): 1024 strips, 8192 chains, 1 GiB; fp32 (32, 512, 8192): 1024
    strips, exactly 512 MiB). Checked through the C ABI (workspace of the tiled size, every
    aggregate published, no overrun), against the oracle on sampled columns, and bit for bit
    against reverse = flip(forward(flip))."""
    shape = (64, 1024, 8192) if dtype == torch.bfloat16 else (32, 512, 8192)
    B, L, D = shape
    gen = torch.Generator(device=DEVICE).manual_seed(9)
    g = (0.99 + 0.01 * torch.rand(shape, generator=gen, device=DEVICE)).to(dtype)
    x = (torch.randn(shape, generator=gen, device=DEVICE) / L).to(dtype)
    assert lib.fpscan_workspace_bytes_cl(B, L, D, D, _CODE[dtype], 0) == (
        tile_geometry(B, L, D, dtype)[2] * 768 + _EXTRA_WORDS * 8)
    out = abi_fwd(lib, g, x, False)
    rows = torch.linspace(0, B - 1, 4).long()
    cols = torch.linspace(0, D - 1, 24).long()
    sel = lambda t: t[rows][:, :, cols].cpu()  # noqa: E731
    check(sel(out), oracle.scan_f64_channel_last(sel(g), sel(x)), dtype, f"large {shape}")
    rev = abi_fwd(lib, g, x, True, ws_check=False)
    mirrored = abi_fwd(lib, g.flip(1).contiguous(), x.flip(1).contiguous(), False,
                       ws_check=False).flip(1)
    assert bits_equal(rev, mirrored)
