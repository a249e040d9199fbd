"""GPU check of the bandwidth probes (include/fpscan_probe.h): every pattern reads every input
byte and writes every output byte, so that its timing is that of the full traffic. Inputs are
small integer patterns; each output must equal the exact 32-bit integer combination."""
import ctypes
import os

import pytest
import torch

import fpscan_amd

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device (MI355X)"),
]


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(os.path.join(os.path.dirname(fpscan_amd.__file__), "libfpscan_hip.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_probe_copy.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, i64, i64,
                                      vp, ctypes.c_size_t, vp]
    lib.fpscan_probe_copy.restype = ctypes.c_int
    lib.fpscan_probe_scratch_bytes.restype = ctypes.c_size_t
    lib.fpscan_probe_lookback_scratch_bytes.argtypes = [i64]
    lib.fpscan_probe_lookback_scratch_bytes.restype = ctypes.c_size_t
    return lib


@pytest.mark.parametrize("pattern", [0, 1, 2, 3, 4, 5],
                         ids=["tiles", "blocks", "rows", "lookback", "rows8", "tiles8"])
@pytest.mark.parametrize("nr,nw", [(2, 1), (3, 2)], ids=["2r1w", "3r2w"])
@pytest.mark.parametrize("tensor_kib,row_kib", [(16, 16), (4096, 128), (49152, 256)])
def test_probe_moves_every_byte(lib, pattern, nr, nw, tensor_kib, row_kib):
    n = tensor_kib * 256  # int32 elements per tensor
    gen = torch.Generator(device="cuda").manual_seed(tensor_kib + 7 * nr)
    src = torch.randint(-1000, 1000, (nr, n), generator=gen, device="cuda", dtype=torch.int32)
    dst = torch.full((nw, n), -7, device="cuda", dtype=torch.int32)
    nbytes = (lib.fpscan_probe_lookback_scratch_bytes(n * 4) if pattern == 3
              else lib.fpscan_probe_scratch_bytes())
    scratch = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    for _ in range(2):  # the tile claims start from a cleared scratch on every call
        st = lib.fpscan_probe_copy(pattern, nr, nw, src.data_ptr(), dst.data_ptr(), n * 4,
                                   row_kib << 10, scratch.data_ptr(), scratch.numel(),
                                   torch.cuda.current_stream().cuda_stream)
        assert st == 0
        torch.cuda.synchronize()
        for o in range(nw):
            want = src[0] + (o + 1) * src[1:].sum(0, dtype=torch.int32)
            assert torch.equal(dst[o], want), f"output {o}"
        dst.fill_(-7)
    if pattern == 3:
        assert scratch[4:8].view(torch.int32).item() == 0, "a look-back wait gave up"


@pytest.mark.parametrize("nr,nw", [(2, 1), (3, 2)], ids=["2r1w", "3r2w"])
@pytest.mark.parametrize("batch,seqlen,row_bytes,strip", [
    (1, 128, 2048, 128),    # 16 chains of one tile: the batch-1 channel-last share's rows
    (3, 256, 512, 256),     # 6 chains: fewer than the 8 claim groups
    (2, 1024, 4096, 128),   # 64 chains of 8 tiles
    (1, 512, 2048, 256),    # fp32 strips, 8 chains of 8 tiles
])
def test_channel_last_probe_moves_every_byte(lib, nr, nw, batch, seqlen, row_bytes, strip):
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_probe_copy_cl.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, i64, i64, i64,
                                         ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fpscan_probe_copy_cl.restype = ctypes.c_int
    n = batch * seqlen * row_bytes // 4
    gen = torch.Generator(device="cuda").manual_seed(n + nr)
    src = torch.randint(-1000, 1000, (nr, n), generator=gen, device="cuda", dtype=torch.int32)
    dst = torch.full((nw, n), -7, device="cuda", dtype=torch.int32)
    scratch = torch.zeros(lib.fpscan_probe_scratch_bytes(), dtype=torch.uint8, device="cuda")
    for _ in range(2):
        st = lib.fpscan_probe_copy_cl(nr, nw, src.data_ptr(), dst.data_ptr(), batch, seqlen,
                                      row_bytes, strip, scratch.data_ptr(), scratch.numel(),
                                      torch.cuda.current_stream().cuda_stream)
        assert st == 0
        torch.cuda.synchronize()
        for o in range(nw):
            want = src[0] + (o + 1) * src[1:].sum(0, dtype=torch.int32)
            assert torch.equal(dst[o], want), f"output {o}"
        dst.fill_(-7)
