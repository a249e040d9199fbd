"""fpscan_scan_fwd_noalloc -- the entry point that allocates nothing (its tiled path keeps its
tile status words and claim counters in a static device array of the library) -- against
fpscan_scan_fwd with a caller-provided workspace, through the C ABI, bit for bit.

Both take the same path for the same problem and tiling mode, and the tiled path composes
each tile's predecessors in a fixed order, so the results must be identical. Two calls follow
each other, the second with a smaller problem, so the second runs on the scratch the first
one left behind.
"""
import ctypes
import os

import pytest
import torch

from conftest import ROOT
from scan_helpers import DEVICE, bits_equal, make_inputs

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]

LIB = os.path.join(ROOT, "fpscan_amd", "libfpscan_hip.so")
CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


@pytest.fixture(scope="module")
def lib():
    import fpscan_amd  # noqa: F401  (torch and the HIP runtime first, as in every GPU test)

    lib = ctypes.CDLL(LIB)
    vp, i64, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.fpscan_scan_fwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, c_int, c_int, vp,
                                    ctypes.c_size_t, vp]
    lib.fpscan_scan_fwd.restype = c_int
    lib.fpscan_scan_fwd_noalloc.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, c_int, c_int,
                                            vp]
    lib.fpscan_scan_fwd_noalloc.restype = c_int
    lib.fpscan_workspace_bytes.argtypes = [i64, i64, i64, c_int, c_int]
    lib.fpscan_workspace_bytes.restype = ctypes.c_size_t
    lib.fpscan_set_tiling.argtypes = [c_int]
    return lib


def _pair(lib, shape, dtype, reverse, seed):
    """(result of fpscan_scan_fwd with a workspace, result of fpscan_scan_fwd_noalloc)."""
    B, D, L = shape
    print(f"noalloc case: shape {shape} {dtype} reverse={reverse}", flush=True)
    g, x = make_inputs(B, D, L, dtype, seed=seed)
    g, x = g.to(DEVICE), x.to(DEVICE)
    want, got = torch.empty_like(x), torch.full_like(x, float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    code = CODE[dtype]
    nb = lib.fpscan_workspace_bytes(B, D, L, code, 0)
    ws = torch.empty(max(nb, 8), dtype=torch.uint8, device=DEVICE)
    assert lib.fpscan_scan_fwd(g.data_ptr(), x.data_ptr(), want.data_ptr(), B, D, L, D * L, L,
                               code, reverse, ws.data_ptr() if nb else None, nb, stream) == 0
    assert lib.fpscan_scan_fwd_noalloc(g.data_ptr(), x.data_ptr(), got.data_ptr(), B, D, L,
                                       D * L, L, code, reverse, stream) == 0
    torch.cuda.synchronize()
    return want, got, nb


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("reverse", [0, 1], ids=["fwd", "rev"])
def test_noalloc_equals_workspace_entry_point_tiled(lib, dtype, reverse):
    """Tiled path forced: 256 rows of 8 (bf16) or 16 (fp32) tiles, then 6 rows of 2 or 4."""
    lib.fpscan_set_tiling(2)
    try:
        for shape, seed in (((4, 64, 65536), 1), ((2, 3, 16384), 2)):
            want, got, nb = _pair(lib, shape, dtype, reverse, seed)
            assert nb > 0, "the case must take the tiled path"
            assert bits_equal(got, want), f"noalloc differs at {shape}"
    finally:
        lib.fpscan_set_tiling(0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_noalloc_equals_workspace_entry_point_automatic(lib, dtype):
    """Automatic path choice: 512 MiB per tensor (tiled), then a small problem (streamed)."""
    shapes = {torch.bfloat16: (4, 1024, 65536), torch.float32: (2, 1024, 65536)}
    for shape, seed, tiled in ((shapes[dtype], 3, True), ((2, 4, 1024), 4, False)):
        want, got, nb = _pair(lib, shape, dtype, 0, seed)
        assert (nb > 0) == tiled
        assert bits_equal(got, want), f"noalloc differs at {shape}"
        del want, got
