"""CPU checks of the drop-in boundary: the C-ABI library and the torch binding load, export
what include/fpscan_hip.h declares, and reject bad arguments before any HIP call.

No kernel is launched here (no GPU in this container): every call below fails validation
first, which the C ABI does before touching the HIP runtime.
"""
import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "fpscan_hip.h")
LIB = os.path.join(ROOT, "fpscan_amd", "libfpscan_hip.so")


def header_functions(path=HEADER):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fpscan_\w+)\s*\(", text, flags=re.M)


def all_headers():
    inc = os.path.join(ROOT, "include")
    return sorted(os.path.join(inc, f) for f in os.listdir(inc) if f.endswith(".h"))


def header_defines():
    text = open(HEADER).read()
    return {m.group(1): int(m.group(2)) for m in
            re.finditer(r"#define\s+(FPSCAN_\w+)\s+(\d+)", text)}


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built; run __graft_entry__.build() first")
    lib = ctypes.CDLL(LIB)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_scan_fwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                    ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fpscan_scan_fwd.restype = ctypes.c_int
    lib.fpscan_scan_bwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                    vp, ctypes.c_size_t, vp]
    lib.fpscan_scan_bwd.restype = ctypes.c_int
    lib.fpscan_strerror.argtypes = [ctypes.c_int]
    lib.fpscan_strerror.restype = ctypes.c_char_p
    lib.fpscan_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int, ctypes.c_int]
    lib.fpscan_workspace_bytes.restype = ctypes.c_size_t
    lib.fpscan_set_launch_override.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.fpscan_set_launch_override.restype = ctypes.c_int
    return lib


def test_header_declares_the_expected_entry_points():
    names = header_functions()
    assert {"fpscan_scan_fwd", "fpscan_scan_bwd", "fpscan_workspace_bytes", "fpscan_strerror",
            "fpscan_abi_version", "fpscan_set_launch_override", "fpscan_set_tiling",
            "fpscan_lookback_overruns", "fpscan_set_lookback_test_hook",
            "fpscan_scan_fwd_noalloc"} <= set(names)


def test_library_exports_every_declared_symbol(lib):
    headers = all_headers()
    assert HEADER in headers and len(headers) >= 2
    for path in headers:
        for name in header_functions(path):
            assert hasattr(lib, name), f"{name} declared in {os.path.basename(path)} but not exported"


def test_probe_rejects_bad_arguments_before_any_launch(lib):
    """The bandwidth probe (include/fpscan_probe.h) validates its arguments on the host."""
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_probe_copy.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, i64, i64,
                                      vp, ctypes.c_size_t, vp]
    lib.fpscan_probe_copy.restype = ctypes.c_int
    lib.fpscan_probe_scratch_bytes.restype = ctypes.c_size_t
    assert lib.fpscan_probe_scratch_bytes() == 8 * 16 * 9
    buf, kib16 = 1 << 20, 16 << 10
    bad = [
        (7, 2, 1, buf, buf, kib16, 0, None, 0),        # unknown pattern
        (3, 2, 1, buf, buf, kib16, kib16, None, 0),    # look-back blocks without scratch
        (1, 2, 2, buf, buf, kib16, 0, None, 0),        # (2, 2) is not a scan's traffic
        (1, 2, 1, None, buf, kib16, 0, None, 0),       # null source
        (1, 2, 1, buf + 8, buf, kib16, 0, None, 0),    # misaligned
        (1, 2, 1, buf, buf, kib16 + 16, 0, None, 0),   # not whole tiles
        (1, 2, 1, buf, buf, (1 << 32) + kib16, 0, None, 0),  # above 4 GiB
        (2, 2, 1, buf, buf, 4 * kib16, 3 * kib16, None, 0),  # rows that do not divide
        (4, 2, 1, buf, buf, 4 * kib16, 3 * kib16, None, 0),  # eight-wave rows likewise
        (4, 2, 1, buf, buf, 4 * kib16, 0, None, 0),    # eight-wave rows without a row length
        (0, 2, 1, buf, buf, kib16, 0, None, 0),        # tiles without scratch
        (5, 2, 1, buf, buf, kib16, 0, None, 0),        # 8 KiB tiles likewise
        (0, 3, 2, buf, buf, kib16, 0, buf, 64),        # scratch too small
    ]
    for args in bad:
        assert lib.fpscan_probe_copy(*args, None) == 1, args
    lib.fpscan_probe_copy_cl.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, i64, i64, i64,
                                         ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fpscan_probe_copy_cl.restype = ctypes.c_int
    scratch = lib.fpscan_probe_scratch_bytes()
    bad_cl = [
        (2, 2, buf, buf, 1, 128, 2048, 128, buf, scratch),     # (2, 2) traffic
        (2, 1, buf, buf, 1, 129, 2048, 128, buf, scratch),     # not whole 128-row tiles
        (2, 1, buf, buf, 1, 64, 2048, 256, buf + 4, scratch),  # misaligned scratch
        (2, 1, buf, buf, 1, 128, 2048, 64, buf, scratch),      # strips of 64 bytes
        (2, 1, buf, buf, 1, 128, 2000, 128, buf, scratch),     # rows not whole strips
        (2, 1, buf, buf, 0, 128, 2048, 128, buf, scratch),     # empty batch
        (3, 2, buf, buf, 1, 128, 2048, 128, None, scratch),    # no scratch
        (3, 2, buf, buf, 1, 128, 2048, 128, buf, 64),          # scratch too small
        (2, 1, buf, buf, 2, 1 << 20, 4096, 128, buf, scratch),  # above 4 GiB
        (2, 1, buf, buf, 1 << 40, 1 << 40, 1 << 40, 128, buf, scratch),  # would overflow
    ]
    for args in bad_cl:
        assert lib.fpscan_probe_copy_cl(*args, None) == 1, args


def test_abi_version_matches_header(lib):
    assert lib.fpscan_abi_version() == header_defines()["FPSCAN_ABI_VERSION"]


def test_strerror_covers_every_status(lib):
    d = header_defines()
    codes = [v for k, v in d.items() if k == "FPSCAN_OK" or k.startswith("FPSCAN_ERR_")]
    texts = {lib.fpscan_strerror(c).decode() for c in codes}
    assert len(texts) == len(codes)  # one distinct message per status
    assert lib.fpscan_strerror(999).decode() == "unknown fpscan status"
    assert "power of 2" in lib.fpscan_strerror(d["FPSCAN_ERR_SEQLEN"]).decode()


def test_workspace_plan(lib):
    lib.fpscan_set_tiling.argtypes = [ctypes.c_int]
    # tiled path: one 8-byte status word per tile of 16 sub-chunks, then an overrun counter
    # and 8 claim counters, each on its own 128-byte line
    extra = 16 * (1 + 8)
    tiles_bf16 = 8 * 1024 * (65536 // 512 // 16)
    assert lib.fpscan_workspace_bytes(8, 1024, 65536, 2, 0) == 8 * (tiles_bf16 + extra)
    assert lib.fpscan_workspace_bytes(8, 1024, 65536, 2, 1) == 8 * (tiles_bf16 + extra)
    tiles_f32 = 8 * 1024 * (65536 // 256 // 16)
    assert lib.fpscan_workspace_bytes(8, 1024, 65536, 0, 1) == 8 * (tiles_f32 + extra)
    assert lib.fpscan_workspace_bytes(8, 1024, 65536, 0, 0) == 8 * (tiles_f32 + extra)
    # small problems and short rows stream rows and need nothing
    assert lib.fpscan_workspace_bytes(2, 256, 1024, 0, 0) == 0
    assert lib.fpscan_workspace_bytes(64, 4096, 256, 0, 0) == 0
    assert lib.fpscan_workspace_bytes(2, 256, 65536, 0, 0) == 0  # 128 MiB per tensor
    # from 256 MiB per tensor the backward tiles rows of 64 KiB or more; the forward waits
    # for 512 MiB, and shorter rows stream in both
    tiles_b2 = 2 * 1024 * (65536 // 512 // 16)
    assert lib.fpscan_workspace_bytes(2, 1024, 65536, 2, 1) == 8 * (tiles_b2 + extra)
    assert lib.fpscan_workspace_bytes(2, 1024, 65536, 2, 0) == 0
    tiles_64k = 4 * 1024 * (32768 // 512 // 16)  # 64 KiB rows
    assert lib.fpscan_workspace_bytes(4, 1024, 32768, 2, 1) == 8 * (tiles_64k + extra)
    assert lib.fpscan_workspace_bytes(4, 1024, 32768, 2, 0) == 0
    assert lib.fpscan_workspace_bytes(8, 1024, 16384, 2, 1) == 0  # 32 KiB rows
    assert lib.fpscan_workspace_bytes(1, 1024, 65536, 2, 1) == 0  # 128 MiB per tensor
    # rows of one tile (16 sub-chunks: bf16 L8192, fp32 L4096) stream up to 1 GiB per tensor,
    # and the 2-byte backward on them at every size
    for code, L in ((2, 8192), (0, 4096)):
        for op in (0, 1):
            assert lib.fpscan_workspace_bytes(32, 1024, L, code, op) == 0  # 512 MiB
            tiled = 8 * (64 * 1024 + extra)
            want = 0 if (code == 2 and op == 1) else tiled
            assert lib.fpscan_workspace_bytes(64, 1024, L, code, op) == want
    assert lib.fpscan_workspace_bytes(0, 4, 65536, 2, 0) == 0
    assert lib.fpscan_workspace_bytes(2, 4, 100, 2, 0) == 0
    try:
        assert lib.fpscan_set_tiling(1) == 0  # row streaming only
        assert lib.fpscan_workspace_bytes(8, 1024, 65536, 2, 0) == 0
        assert lib.fpscan_set_tiling(2) == 0  # tiled whenever the row allows
        assert lib.fpscan_workspace_bytes(1, 2, 8192, 2, 0) == 8 * (2 * 1 + extra)
        assert lib.fpscan_workspace_bytes(1, 2, 4096, 2, 0) == 0  # < 16 sub-chunks per row
        assert lib.fpscan_set_tiling(3) != 0
    finally:
        lib.fpscan_set_tiling(0)


FAKE = 0x10000  # 16-byte aligned, never dereferenced: every call below fails validation


@pytest.mark.parametrize("seqlen", [0, 16, 30, 48, 100, 131072])
def test_bad_seqlen_rejected(lib, seqlen):
    d = header_defines()
    assert lib.fpscan_scan_fwd(FAKE, FAKE, FAKE, 2, 4, seqlen, 4 * seqlen, seqlen, 0, 0,
                               None, 0, None) == d["FPSCAN_ERR_SEQLEN"]
    assert lib.fpscan_scan_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 4, seqlen, 4 * seqlen, seqlen,
                               0, None, 0, None) == d["FPSCAN_ERR_SEQLEN"]


def test_bad_dtype_rejected(lib):
    assert lib.fpscan_scan_fwd(FAKE, FAKE, FAKE, 2, 4, 64, 256, 64, 3, 0, None, 0, None) == \
        header_defines()["FPSCAN_ERR_DTYPE"]


def test_bad_shape_rejected(lib):
    d = header_defines()
    assert lib.fpscan_scan_fwd(FAKE, FAKE, FAKE, -1, 4, 64, 256, 64, 0, 0, None, 0, None) == \
        d["FPSCAN_ERR_SHAPE"]
    # rows overlapping: stride_d smaller than seqlen
    assert lib.fpscan_scan_fwd(FAKE, FAKE, FAKE, 1, 4, 64, 256, 32, 0, 0, None, 0, None) == \
        d["FPSCAN_ERR_SHAPE"]
    # sizes whose row count or element span would wrap around a 64-bit integer, or exceed
    # 2^48 bytes: refused, never launched
    big = 1 << 40
    for args in ((big, big, 64, big * 64, 64), (3, 4, 64, (1 << 62), 64),
                 (2, big, 64, big * 64, 64), ((1 << 62), 2, 64, 128, 64)):
        assert lib.fpscan_scan_fwd(FAKE, FAKE, FAKE, *args, 0, 0, None, 0, None) == \
            d["FPSCAN_ERR_SHAPE"], args
        assert lib.fpscan_workspace_bytes(args[0], args[1], args[2], 0, 0) == 0, args


def test_misaligned_rejected(lib):
    d = header_defines()
    assert lib.fpscan_scan_fwd(FAKE + 4, FAKE, FAKE, 2, 4, 64, 256, 64, 0, 0, None, 0, None) \
        == d["FPSCAN_ERR_ALIGN"]
    # fp16 row stride of 36 elements = 72 bytes is not a multiple of 16
    assert lib.fpscan_scan_fwd(FAKE, FAKE, FAKE, 1, 4, 32, 144, 36, 1, 0, None, 0, None) == \
        d["FPSCAN_ERR_ALIGN"]


def test_null_pointer_rejected_and_empty_problem_accepted(lib):
    d = header_defines()
    assert lib.fpscan_scan_fwd(None, FAKE, FAKE, 2, 4, 64, 256, 64, 0, 0, None, 0, None) == \
        d["FPSCAN_ERR_NULL"]
    # zero rows: nothing to do, no pointer is needed and nothing is launched
    assert lib.fpscan_scan_fwd(None, None, None, 0, 4, 64, 256, 64, 0, 0, None, 0, None) == 0
    assert lib.fpscan_scan_bwd(None, None, None, None, None, 2, 0, 64, 0, 64, 2, None, 0,
                               None) == 0


def test_noalloc_rejects_problems_beyond_its_scratch(lib):
    """fpscan_scan_fwd_noalloc's static scratch holds 262144 tiles; a problem whose tiled plan
    needs more fails with FPSCAN_ERR_SCRATCH before any HIP call (fake pointers are safe)."""
    d = header_defines()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_scan_fwd_noalloc.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                            ctypes.c_int, vp]
    lib.fpscan_scan_fwd_noalloc.restype = ctypes.c_int
    # fp32 (32, 1024, 65536): 32768 rows x 16 tiles = 524288 tiles, tiled by default
    assert lib.fpscan_scan_fwd_noalloc(FAKE, FAKE, FAKE, 32, 1024, 65536, 1024 * 65536, 65536,
                                       0, 0, None) == d["FPSCAN_ERR_SCRATCH"]
    assert lib.fpscan_scan_fwd_noalloc(FAKE, FAKE, FAKE, 2, 4, 100, 400, 100, 0, 0,
                                       None) == d["FPSCAN_ERR_SEQLEN"]
    assert "262144 tiles" in lib.fpscan_strerror(d["FPSCAN_ERR_SCRATCH"]).decode()


def test_lookback_test_hook_validation(lib):
    lib.fpscan_set_lookback_test_hook.argtypes = [ctypes.c_int64, ctypes.c_int]
    try:
        assert lib.fpscan_set_lookback_test_hook(-1, -5) != 0  # a negative poll bound
        assert lib.fpscan_set_lookback_test_hook(3, 16) == 0
    finally:
        assert lib.fpscan_set_lookback_test_hook(-1, 0) == 0  # the defaults


def test_lookback_overruns_rejects_null(lib):
    lib.fpscan_lookback_overruns.argtypes = [ctypes.c_void_p]
    assert lib.fpscan_lookback_overruns(None) == header_defines()["FPSCAN_ERR_NULL"]


def test_launch_override_validation(lib):
    d = header_defines()
    assert lib.fpscan_set_launch_override(3, 0) == d["FPSCAN_ERR_SHAPE"]
    assert lib.fpscan_set_launch_override(0, 5) == d["FPSCAN_ERR_SHAPE"]
    assert lib.fpscan_set_launch_override(16, 3) == 0
    assert lib.fpscan_set_launch_override(4, 2) == 0
    assert lib.fpscan_set_launch_override(0, 0) == 0


# ---------------------------------------------------------------- torch binding
def test_binding_loads_and_exposes_the_reference_surface():
    from fpscan_amd import ops

    ext = ops._load_extension()
    assert ext.__file__.startswith(os.path.join(ROOT, "fpscan_amd"))
    for name in ("fullscan_forward", "fullscan_backward", "set_launch_override"):
        assert hasattr(ext, name)


def test_public_api_names():
    import fpscan_amd

    assert set(fpscan_amd.__all__) >= {"pscan", "scan_forward", "PScan"}


@pytest.mark.parametrize("call", ["forward", "reverse", "pscan", "backward"])
def test_cpu_tensors_raise_runtime_error(call):
    import fpscan_amd

    g, x = torch.rand(2, 4, 64), torch.rand(2, 4, 64)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        if call == "forward":
            fpscan_amd.scan_forward(g, x)
        elif call == "reverse":
            fpscan_amd.scan_forward(g, x, reverse=True)
        elif call == "pscan":
            fpscan_amd.pscan(g, x)
        else:
            fpscan_amd.scan_backward(g, x, x)


def test_missing_extension_raises_import_error(monkeypatch):
    """fpscan/ops.py:40-44: no importable candidate -> ImportError naming each failure."""
    from fpscan_amd import ops

    monkeypatch.setattr(ops, "_ext", None)
    monkeypatch.setattr(ops, "_EXT_CANDIDATES", ("fpscan_amd._no_such_module",))
    with pytest.raises(ImportError, match="_no_such_module"):
        ops.scan_forward(torch.rand(1, 1, 32), torch.rand(1, 1, 32))


# ---------------------------------------------------------------- channel-last C ABI
@pytest.fixture(scope="module")
def cl_lib(lib):
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.fpscan_scan_fwd_cl.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                       ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fpscan_scan_bwd_cl.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                       vp, ctypes.c_size_t, vp]
    lib.fpscan_workspace_bytes_cl.argtypes = [i64, i64, i64, i64, ctypes.c_int, ctypes.c_int]
    lib.fpscan_workspace_bytes_cl.restype = ctypes.c_size_t
    return lib


def test_channel_last_validation(cl_lib):
    d = header_defines()
    f = cl_lib.fpscan_scan_fwd_cl
    # (batch, seqlen, dim) = (2, 100, 64), packed strides (stride_b = 6400, stride_t = 64)
    assert f(FAKE, FAKE, FAKE, 2, 100, 64, 6400, 64, 3, 0, None, 0, None) == d["FPSCAN_ERR_DTYPE"]
    assert f(FAKE, FAKE, FAKE, -1, 100, 64, 6400, 64, 0, 0, None, 0, None) == d["FPSCAN_ERR_SHAPE"]
    assert f(FAKE, FAKE, FAKE, 2, 100, 64, 6400, 32, 0, 0, None, 0, None) == d["FPSCAN_ERR_SHAPE"]
    assert f(FAKE, FAKE, FAKE, 2, 100, 64, 100, 64, 0, 0, None, 0, None) == d["FPSCAN_ERR_SHAPE"]
    assert f(FAKE, FAKE, FAKE, 2, 100, 62, 6200, 62, 0, 0, None, 0, None) == d["FPSCAN_ERR_ALIGN"]
    assert f(FAKE, FAKE, FAKE, 2, 100, 60, 6000, 60, 1, 0, None, 0, None) == d["FPSCAN_ERR_ALIGN"]
    assert f(FAKE + 8, FAKE, FAKE, 2, 100, 64, 6400, 64, 0, 0, None, 0, None) == \
        d["FPSCAN_ERR_ALIGN"]
    assert f(None, FAKE, FAKE, 2, 100, 64, 6400, 64, 0, 0, None, 0, None) == d["FPSCAN_ERR_NULL"]
    assert f(None, None, None, 0, 100, 64, 6400, 64, 0, 0, None, 0, None) == 0  # empty
    assert f(None, None, None, 2, 0, 64, 0, 64, 0, 0, None, 0, None) == 0
    # spans that would wrap around a 64-bit integer or exceed 2^48 bytes
    assert f(FAKE, FAKE, FAKE, 1 << 40, 1 << 30, 64, 64 << 30, 64, 0, 0, None, 0, None) == \
        d["FPSCAN_ERR_SHAPE"]
    assert f(FAKE, FAKE, FAKE, 3, 100, 64, 1 << 62, 64, 0, 0, None, 0, None) == \
        d["FPSCAN_ERR_SHAPE"]
    b = cl_lib.fpscan_scan_bwd_cl
    assert b(FAKE, FAKE, FAKE, FAKE, None, 2, 100, 64, 6400, 64, 0, None, 0, None) == \
        d["FPSCAN_ERR_NULL"]


def _cl_tiled_bytes(batch, seqlen, dim, itemsize):
    """Tiled channel-last workspace: tiles of 64 columns x 16 * (16 / itemsize) steps, per
    tile 64 aggregate words (8 bytes) and 64 end values (4 bytes), then 144 extra words."""
    steps = 16 * (16 // itemsize)
    ntiles = batch * -(-dim // 64) * -(-seqlen // steps)
    return ntiles * 64 * 12 + 144 * 8


def test_channel_last_workspace_plan(cl_lib):
    """Automatic choice: one pass when batch x strips (64 16-byte vectors each) reaches 512
    and a tensor is below 512 MiB; otherwise the tiled single pass (tiles of 64 columns by
    16 x 16/itemsize steps) when seqlen spans more than one tile, else segments of about 1024
    steps, more if needed for 1024 wave tasks, never below 64 steps, with one (A, B) pair of
    8 bytes per segment per column (or the one pass, with 512 strips or more)."""
    w = cl_lib.fpscan_workspace_bytes_cl
    assert w(64, 256, 4096, 4096, 0, 0) == 0  # config 5 in channel-last form: 1024 strips
    assert w(64, 256, 4096, 4096, 2, 0) == 0  # bf16, 512 strips, 128 MiB: one pass
    assert w(32, 511, 8192, 8192, 0, 0) == 0  # fp32, 1024 strips, just below 512 MiB
    # 512 MiB and more per tensor: tiled whatever the strips
    assert w(32, 512, 8192, 8192, 0, 0) == _cl_tiled_bytes(32, 512, 8192, 4)
    assert w(64, 1024, 8192, 8192, 0, 0) == _cl_tiled_bytes(64, 1024, 8192, 4)  # 2048 strips
    assert w(16, 4096, 8192, 8192, 0, 0) == _cl_tiled_bytes(16, 4096, 8192, 4)  # 512 strips
    # ... unless seqlen fits one tile: fp32 (8192, 64, 1024), 2 GiB, one pass
    assert w(8192, 64, 1024, 1024, 0, 0) == 0
    assert w(1, 100, 64, 64, 0, 0) == _cl_tiled_bytes(1, 100, 64, 4)  # two 64-step tiles
    # bf16 (8, 65536, 1024): 16 strips, 128 chains -> tiled, 512 tiles of 128 steps per chain
    assert w(8, 65536, 1024, 1024, 2, 0) == _cl_tiled_bytes(8, 65536, 1024, 2) == 50332800
    assert w(8, 65536, 1024, 1024, 2, 1) == _cl_tiled_bytes(8, 65536, 1024, 2)
    # fp32 (4, 4096, 8192): 128 strips, 512 chains -> tiled (64-step tiles)
    assert w(4, 4096, 8192, 8192, 0, 0) == _cl_tiled_bytes(4, 4096, 8192, 4)
    # few chains: bf16 (4, 8192, 512) 32 chains of 64 tiles, fp32 (1, 1000, 64) one of 16
    assert w(4, 8192, 512, 512, 2, 0) == _cl_tiled_bytes(4, 8192, 512, 2) == 32 * 64 * 768 + 1152
    assert w(1, 1000, 64, 64, 0, 0) == _cl_tiled_bytes(1, 1000, 64, 4) == 16 * 768 + 1152
    # seqlen within one tile: bf16 (1, 128, 64) -> 2 segments of 64 steps (seqlen / 64)
    assert w(1, 128, 64, 64, 2, 0) == 2 * 1 * 64 * 8
    assert w(1, 64, 64, 64, 0, 0) == 0  # fp32, one tile and too short to cut: one pass
    assert w(1, 100, 64, 64, 0, 7) == 0  # unknown op
    assert w(1, 100, 64, 64, 5, 0) == 0  # unknown dtype
    assert w(1, 100, 64, 32, 0, 0) == 0  # stride_t < dim


def test_channel_last_workspace_plan_forced_modes(cl_lib):
    """fpscan_set_tiling(1): never tiled (segments as above); (2): tiled whenever the
    workspace fits, whatever the chain count."""
    w = cl_lib.fpscan_workspace_bytes_cl
    try:
        assert cl_lib.fpscan_set_tiling(1) == 0
        assert w(8, 65536, 1024, 1024, 2, 0) == 64 * 8 * 1024 * 8  # 64 segments of 1024
        assert w(4, 4096, 8192, 8192, 0, 0) == 8 * 4 * 8192 * 8  # 8 segments of 512
        # segments capped by seqlen / 64: bf16 (4, 8192, 512) -> 128 of 64 steps,
        # fp32 (1, 1000, 64) -> 15 of 67 steps
        assert w(4, 8192, 512, 512, 2, 0) == 128 * 4 * 512 * 8
        assert w(1, 1000, 64, 64, 0, 0) == 15 * 1 * 64 * 8
        assert w(64, 256, 4096, 4096, 0, 0) == 0
        assert cl_lib.fpscan_set_tiling(2) == 0
        assert w(1, 1000, 64, 64, 0, 0) == _cl_tiled_bytes(1, 1000, 64, 4) == 16 * 768 + 1152
        assert w(64, 256, 4096, 4096, 0, 0) == _cl_tiled_bytes(64, 256, 4096, 4)
        assert w(3, 1, 200, 200, 2, 1) == _cl_tiled_bytes(3, 1, 200, 2)
        # bf16 rows 2^24 bytes apart: a tile's 130 rows exceed one 2 GiB buffer range, so
        # segments (at most 126 rows each: 5 of 103 steps) even when tiling is forced
        assert w(1, 512, 1 << 23, 1 << 23, 2, 0) == 5 * (1 << 23) * 8
    finally:
        cl_lib.fpscan_set_tiling(0)


# ---------------------------------------------------------------- dimwise C ABI
def test_dimwise_groups_and_validation(lib):
    d = header_defines()
    lib.fpscan_dimwise_groups.argtypes = [ctypes.c_int64]
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    f = lib.fpscan_dimwise_fwd
    f.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, ctypes.c_int, vp]
    # G = W * C per seqlen (dimwise_scan_final.cu:408-572); 32 and non-powers rejected
    want = {64: 2, 128: 4, 256: 8, 512: 16, 1024: 16, 2048: 32, 4096: 32, 8192: 64,
            16384: 128, 32768: 256, 65536: 512, 32: 0, 96: 0, 131072: 0}
    assert {L: lib.fpscan_dimwise_groups(L) for L in want} == want
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 4, 32, 0, None) == d["FPSCAN_ERR_SEQLEN"]
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 4, 64, 3, None) == d["FPSCAN_ERR_DTYPE"]
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, -1, 4, 64, 0, None) == d["FPSCAN_ERR_SHAPE"]
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 40, 1 << 40, 64, 0, None) == d["FPSCAN_ERR_SHAPE"]
    assert f(FAKE, None, FAKE, FAKE, FAKE, 2, 4, 64, 0, None) == d["FPSCAN_ERR_NULL"]
    assert f(FAKE + 4, FAKE, FAKE, FAKE, FAKE, 2, 4, 64, 0, None) == d["FPSCAN_ERR_ALIGN"]
    assert f(None, None, None, None, None, 0, 4, 64, 0, None) == 0  # empty


def test_dimwise_workspace_and_validation(lib):
    """fpscan_dimwise_workspace_bytes: one status word per 16 KiB tile (two chunks of 4096
    elements of a 2-byte type, one of fp32) plus the counters when the tiled path is taken
    (seqlen >= 8192, tensors below 4 GiB; automatically for rows of 64 KiB or more from 384
    MiB per tensor), else 0;
    fpscan_dimwise_fwd_ws validates like fpscan_dimwise_fwd and checks the workspace's
    alignment before any launch."""
    d = header_defines()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    wb = lib.fpscan_dimwise_workspace_bytes
    wb.argtypes = [i64, i64, i64, ctypes.c_int]
    wb.restype = ctypes.c_size_t
    lib.fpscan_set_tiling.argtypes = [ctypes.c_int]
    extra = 16 * 9  # overrun word and claim counters, as the row scan's
    try:
        assert wb(8, 1024, 65536, 2) == (8192 * 8 + extra) * 8    # bf16: 8 tiles per row
        assert wb(8, 1024, 65536, 0) == (8192 * 16 + extra) * 8   # fp32: 16
        assert wb(16, 1024, 65536, 0) == 0                         # 4 GiB: row kernel
        assert wb(1, 1024, 65536, 2) == 0                          # 128 MiB: row kernel
        assert wb(2, 1024, 65536, 2) == 0                          # 256 MiB: row kernel
        assert wb(3, 1024, 65536, 2) == (3072 * 8 + extra) * 8    # 384 MiB: tiled
        assert wb(8, 1024, 32768, 2) == (8192 * 4 + extra) * 8    # 64 KiB rows: tiled
        assert wb(32, 1024, 16384, 2) == 0                         # 32 KiB rows: row kernel
        assert wb(8, 1024, 4096, 2) == 0                           # one chunk per row
        for bad in [(8, 1024, 65536, 3), (8, 1024, 96, 2), (-1, 4, 65536, 2),
                    (1 << 40, 1 << 40, 65536, 2)]:
            assert wb(*bad) == 0, bad
        assert lib.fpscan_set_tiling(2) == 0
        assert wb(2, 4, 8192, 2) == (8 + extra) * 8                # one tile per row
        assert wb(2, 4, 8192, 0) == (16 + extra) * 8               # fp32: two
        assert wb(2, 4, 4096, 2) == 0
        assert lib.fpscan_set_tiling(1) == 0
        assert wb(8, 1024, 65536, 2) == 0
    finally:
        lib.fpscan_set_tiling(0)
    f = lib.fpscan_dimwise_fwd_ws
    f.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, ctypes.c_int, vp, ctypes.c_size_t, vp]
    ws = 1 << 20
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 4, 32, 0, FAKE, ws, None) == d["FPSCAN_ERR_SEQLEN"]
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 4, 8192, 3, FAKE, ws, None) == d["FPSCAN_ERR_DTYPE"]
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 40, 1 << 40, 8192, 0, FAKE, ws,
             None) == d["FPSCAN_ERR_SHAPE"]
    assert f(FAKE, FAKE, None, FAKE, FAKE, 2, 4, 8192, 0, FAKE, ws, None) == d["FPSCAN_ERR_NULL"]
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 4, 8192, 0, FAKE + 4, ws,
             None) == d["FPSCAN_ERR_ALIGN"]
    assert f(None, None, None, None, None, 0, 4, 8192, 0, None, 0, None) == 0  # empty
