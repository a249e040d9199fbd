"""GPU parity tests of the channel-last scan ((batch, seqlen, dim) tensors scanned along
seqlen) against the CPU oracle (oracle.scan_f64_channel_last / scan_bwd_f64_channel_last,
pinned by tests/test_oracle.py).

The reference has no such entry point; its README.md:94-99 transposes in and out around
pscan. So besides the oracle, every result is also compared with the row-major HIP path on the
transposed tensors: within the north-star tolerance on random data, and bit for bit on integer
data, where every partial result is exact in any association order.

Covered: forward, reverse and the fused backward in every dtype; the automatic choice (which
takes the tiled look-back, tests/test_scan_cl_tiled_gpu.py, wherever one pass per strip lacks
strips), the one-pass and the segmented (aggregate, carry, apply) paths, the last two forced
through the C ABI with the tiled look-back switched off (fpscan_set_tiling(1)); ragged and
non-power-of-two shapes, seqlen 1, partial strips, empty tensors, in-place use, the ignored
first gate, validation errors, autograd, and the channel-last forms of benchmark configs 4 and
5 at their real shapes.
"""
import contextlib
import ctypes
import os

import numpy as np
import pytest
import torch

import fpscan_amd
import oracle
from fpscan_amd.ops import set_tiling
from scan_helpers import DEVICE, DTYPES, NORM_TOL, bits_equal, check

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]

_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def cl_inputs(batch, seqlen, dim, dtype, seed=0):
    """test_fpscan.py:25-29 distributions in (batch, seqlen, dim) layout."""
    gen = torch.Generator().manual_seed(seed)
    gates = 0.99 + 0.01 * torch.rand(batch, seqlen, dim, generator=gen)
    tokens = torch.randn(batch, seqlen, dim, generator=gen) / max(seqlen, 1)
    return gates.to(dtype).contiguous(), tokens.to(dtype).contiguous()


def to_rows(t):
    return t.transpose(1, 2).contiguous()


@contextlib.contextmanager
def tiling(mode):
    """fpscan_set_tiling(mode) for the block (process-wide), automatic again afterwards."""
    set_tiling(mode)
    try:
        yield
    finally:
        set_tiling(0)


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
    return lib


def abi_fwd(lib, g, x, reverse, segmented):
    """The C ABI with (segmented, the tiled look-back off) or without (one pass per strip) the
    workspace."""
    B, L, D = x.shape
    out = torch.empty_like(x)
    with tiling(1):
        nbytes = lib.fpscan_workspace_bytes_cl(B, L, D, D, _CODE[x.dtype], 0) if segmented else 0
        ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=DEVICE)
        st = lib.fpscan_scan_fwd_cl(g.data_ptr(), x.data_ptr(), out.data_ptr(), B, L, D, L * D,
                                    D, _CODE[x.dtype], int(reverse),
                                    ws.data_ptr() if nbytes else None, nbytes,
                                    torch.cuda.current_stream().cuda_stream)
    assert st == 0
    return out, nbytes


def abi_bwd(lib, g, y, go, segmented):
    B, L, D = g.shape
    gg, gx = torch.empty_like(g), torch.empty_like(g)
    with tiling(1):
        nbytes = lib.fpscan_workspace_bytes_cl(B, L, D, D, _CODE[g.dtype], 1) if segmented else 0
        ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=DEVICE)
        st = lib.fpscan_scan_bwd_cl(g.data_ptr(), y.data_ptr(), go.data_ptr(), gg.data_ptr(),
                                    gx.data_ptr(), B, L, D, L * D, D, _CODE[g.dtype],
                                    ws.data_ptr() if nbytes else None, nbytes,
                                    torch.cuda.current_stream().cuda_stream)
    assert st == 0
    return gg, gx, nbytes


SHAPES = [
    (2, 64, 64),      # partial strip (64 of 256/512 columns), one pass
    (3, 1000, 40),    # seqlen not a power of two, dim not a multiple of a strip
    (1, 1, 256),      # one time step
    (4, 300, 520),    # tiled or segmented, ragged last tile or segment
    (2, 4096, 1024),  # tiled or segmented, several strips
    (1, 65536, 64),   # long and narrow: one chain of many tiles, or many segments
]
PATHS = {"auto": 0, "no-tiles": 1}  # fpscan_set_tiling modes


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("path", PATHS)
def test_forward_and_reverse_match_oracle(path, dtype, shape):
    g, x = cl_inputs(*shape, dtype, seed=sum(shape))
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    for rev in (False, True):
        with tiling(PATHS[path]):
            out = fpscan_amd.scan_forward_channel_last(gd, xd, reverse=rev)
        assert out.shape == x.shape and out.dtype == dtype
        check(out, oracle.scan_f64_channel_last(g, x, rev), dtype, f"cl {shape} rev={rev}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("path", PATHS)
def test_backward_matches_oracle(path, dtype, shape):
    g, x = cl_inputs(*shape, dtype, seed=sum(shape) + 1)
    go = torch.randn(shape, generator=torch.Generator().manual_seed(3)).to(dtype)
    gd = g.to(DEVICE)
    with tiling(PATHS[path]):
        y = fpscan_amd.scan_forward_channel_last(gd, x.to(DEVICE))
        gg, gx = fpscan_amd.scan_backward_channel_last(gd, y, go.to(DEVICE))
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, y.cpu(), go)
    check(gx, gx_ref, dtype, f"cl {shape} grad_tokens")
    check(gg, gg_ref, dtype, f"cl {shape} grad_gates")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_one_pass_and_segmented_paths_match_oracle(lib, dtype):
    shape = (2, 2048, 256)  # 2-4 strips in all: segmented when the tiled look-back is off
    g, x = cl_inputs(*shape, dtype, seed=11)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    go = torch.randn(shape, generator=torch.Generator().manual_seed(4)).to(dtype)
    for rev in (False, True):
        want = oracle.scan_f64_channel_last(g, x, rev)
        seg, nbytes = abi_fwd(lib, gd, xd, rev, segmented=True)
        assert nbytes > 0
        one, _ = abi_fwd(lib, gd, xd, rev, segmented=False)
        check(seg, want, dtype, f"segmented rev={rev}")
        check(one, want, dtype, f"one pass rev={rev}")
    y = fpscan_amd.scan_forward_channel_last(gd, xd)
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, y.cpu(), go)
    for segmented in (True, False):
        gg, gx, _ = abi_bwd(lib, gd, y, go.to(DEVICE), segmented)
        check(gx, gx_ref, dtype, f"grad_tokens segmented={segmented}")
        check(gg, gg_ref, dtype, f"grad_gates segmented={segmented}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_exact_on_integer_data_and_equal_to_row_path(lib, dtype):
    """Gates in {0, 1} and small integer tokens: every partial result is exact, so the
    channel-last kernels (both paths) and the row-major kernel on the transposed tensors must
    agree bit for bit with the oracle."""
    gen = torch.Generator().manual_seed(21)
    shape = (2, 4096, 512)
    g = (torch.randint(0, 16, shape, generator=gen) > 0).to(dtype)
    x = torch.randint(-3, 4, shape, generator=gen).to(dtype)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    for rev in (False, True):
        want = torch.from_numpy(oracle.scan_f64_channel_last(g, x, rev))
        if dtype != torch.float32 and want.abs().max() >= 256:
            continue  # not exact in 8-bit mantissas
        seg, _ = abi_fwd(lib, gd, xd, rev, segmented=True)
        one, _ = abi_fwd(lib, gd, xd, rev, segmented=False)
        rows = fpscan_amd.scan_forward(to_rows(gd), to_rows(xd), reverse=rev)
        assert bits_equal(seg.cpu(), want.to(dtype))
        assert bits_equal(one.cpu(), want.to(dtype))
        assert bits_equal(to_rows(rows).cpu(), want.to(dtype))


def test_seqlen_one_is_tokens_and_gate_ignored():
    g = torch.full((2, 1, 64), float("nan"), device=DEVICE)
    x = torch.randn(2, 1, 64, device=DEVICE)
    assert torch.equal(fpscan_amd.scan_forward_channel_last(g, x), x)
    assert torch.equal(fpscan_amd.scan_forward_channel_last(g, x, reverse=True), x)


@pytest.mark.parametrize("shape", [(1, 200, 64), (2, 4096, 256)], ids=str)
def test_first_gate_nan_does_not_propagate(shape):
    g, x = cl_inputs(*shape, torch.float32, seed=2)
    for rev in (False, True):
        gn = g.clone()
        gn[:, -1 if rev else 0, :] = float("nan")
        out = fpscan_amd.scan_forward_channel_last(gn.to(DEVICE), x.to(DEVICE), reverse=rev)
        assert torch.isfinite(out).all()
        check(out, oracle.scan_f64_channel_last(g, x, rev), torch.float32, f"nan gate rev={rev}")


def test_out_parameter_and_in_place():
    g, x = cl_inputs(2, 500, 128, torch.float32, seed=9)
    gd, xd = g.to(DEVICE), x.to(DEVICE)
    want = fpscan_amd.scan_forward_channel_last(gd, xd)
    out = torch.empty_like(xd)
    assert fpscan_amd.scan_forward_channel_last(gd, xd, out=out) is out
    assert torch.equal(out, want)
    xi = xd.clone()
    fpscan_amd.scan_forward_channel_last(gd, xi, out=xi)
    assert torch.equal(xi, want)


def test_empty_tensors():
    for shape in [(0, 64, 64), (2, 0, 64), (2, 64, 0)]:
        g = torch.rand(shape, device=DEVICE)
        out = fpscan_amd.scan_forward_channel_last(g, g.clone())
        assert out.shape == shape
        gg, gx = fpscan_amd.scan_backward_channel_last(g, g.clone(), g.clone())
        assert gg.shape == shape and gx.shape == shape


def test_validation_errors():
    x = torch.rand(2, 64, 64, device=DEVICE)
    with pytest.raises(RuntimeError, match="multiple of 4"):
        fpscan_amd.scan_forward_channel_last(x[..., :62].contiguous(), x[..., :62].contiguous())
    h = x.half()
    with pytest.raises(RuntimeError, match="multiple of 8"):
        fpscan_amd.scan_forward_channel_last(h[..., :60].contiguous(), h[..., :60].contiguous())
    with pytest.raises(RuntimeError, match="contiguous"):
        fpscan_amd.scan_forward_channel_last(x.transpose(1, 2), x.transpose(1, 2))
    with pytest.raises(RuntimeError, match="dtype"):
        fpscan_amd.scan_forward_channel_last(x, x.half())
    with pytest.raises(RuntimeError, match="shape"):
        fpscan_amd.scan_forward_channel_last(x, x[:1].contiguous())
    with pytest.raises(RuntimeError, match="alias"):
        fpscan_amd.scan_backward_channel_last(x, x.clone(), x.clone(), grad_gates=x)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_autograd_matches_oracle(dtype):
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


def test_config5_channel_last_b64_l256_d4096():
    """Config 5 (fp32 B64 D4096 L256) in its transposed (batch, seqlen, dim) form, without the
    transposes."""
    import bench

    gr, xr, gor = bench.make_inputs(64, 4096, 256, torch.float32, "sigmoid", seed=5,
                                    device=DEVICE)
    g, x, go = to_rows(gr), to_rows(xr), to_rows(gor)  # (batch, seqlen, dim)
    out = fpscan_amd.scan_forward_channel_last(g, x)
    rows = fpscan_amd.scan_forward(gr, xr)
    assert oracle.normwise_error(out, to_rows(rows)) <= NORM_TOL[torch.float32]
    cols = torch.linspace(0, 4095, 24).long()
    sel = lambda t: t[:8][:, :, cols].cpu()  # noqa: E731
    check(sel(out), oracle.scan_f64_channel_last(sel(g), sel(x)), torch.float32, "c5 cl")
    gg, gx = fpscan_amd.scan_backward_channel_last(g, out, go)
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(sel(g), sel(out), sel(go))
    check(sel(gx), gx_ref, torch.float32, "c5 cl grad_tokens")
    check(sel(gg), gg_ref, torch.float32, "c5 cl grad_gates")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_config4_channel_last_b8_l65536_d1024(dtype):
    """Headline shape in (batch, seqlen, dim) layout: size-independent properties over the
    whole tensor, the oracle on sampled columns."""
    import bench

    gr, xr, gor = bench.make_inputs(8, 1024, 65536, dtype, "mamba", seed=7, device=DEVICE)
    g, x, go = to_rows(gr), to_rows(xr), to_rows(gor)
    del gr, xr, gor
    out = fpscan_amd.scan_forward_channel_last(g, x)
    # reverse == flip(forward(flip)) bit for bit: the tiles divide seqlen evenly, so the
    # reverse pass runs exactly the mirrored operations
    rev = fpscan_amd.scan_forward_channel_last(g, x, reverse=True)
    fwd_of_flip = fpscan_amd.scan_forward_channel_last(g.flip(1).contiguous(),
                                                       x.flip(1).contiguous())
    assert bits_equal(rev, fwd_of_flip.flip(1))
    del rev, fwd_of_flip
    cols = torch.linspace(0, 1023, 16).long()
    sel = lambda t: t[:, :, cols].cpu()  # noqa: E731
    check(sel(out), oracle.scan_f64_channel_last(sel(g), sel(x)), dtype, "c4 cl")
    gg, gx = fpscan_amd.scan_backward_channel_last(g, out, go)
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(sel(g), sel(out), sel(go))
    check(sel(gx), gx_ref, dtype, "c4 cl grad_tokens")
    check(sel(gg), gg_ref, dtype, "c4 cl grad_gates")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("segmented", [False, True], ids=["one-pass", "segmented"])
def test_padded_strides_through_the_c_abi(lib, dtype, segmented):
    """(batch, seqlen, dim) views of a larger buffer: stride_t = dim + pad, stride_b = seqlen *
    stride_t + pad2; the padding must come back untouched."""
    B, L, D = 2, 3000, 96
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
    with tiling(1):
        nb = lib.fpscan_workspace_bytes_cl(B, L, D, st, code, 0) if segmented else 0
        ws = torch.empty(max(nb, 8), dtype=torch.uint8, device=DEVICE)
        assert (nb > 0) == segmented
        assert lib.fpscan_scan_fwd_cl(gb.data_ptr(), xb.data_ptr(), outb.data_ptr(), B, L, D, sb,
                                      st, code, 0, ws.data_ptr() if nb else None, nb, stream) == 0
        assert lib.fpscan_scan_bwd_cl(gb.data_ptr(), outb.data_ptr(), gob.data_ptr(),
                                      ggb.data_ptr(), gxb.data_ptr(), B, L, D, sb, st, code,
                                      ws.data_ptr() if nb else None, nb, stream) == 0
    torch.cuda.synchronize()
    out = view(outb).cpu()
    check(out, oracle.scan_f64_channel_last(g, x), dtype, "cl strided fwd")
    gg_ref, gx_ref = oracle.scan_bwd_f64_channel_last(g, out, go)
    check(view(gxb).cpu(), gx_ref, dtype, "cl strided grad_tokens")
    check(view(ggb).cpu(), gg_ref, dtype, "cl strided grad_gates")
    mask = torch.ones(B * sb, dtype=torch.bool)
    mask.as_strided((B, L, D), (sb, st, 1)).fill_(False)
    for buf in (outb, ggb, gxb):
        assert (buf.cpu()[mask] == -3.0).all(), "padding was written"
