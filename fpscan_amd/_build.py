"""In-tree build of the HIP scan library and its torch binding.

  fpscan_amd/libfpscan_hip.so   hipcc --offload-arch=gfx950: kernels + the C ABI
                                (include/fpscan_hip.h); no torch dependency
  fpscan_amd/_C<EXT_SUFFIX>     g++: the pybind11/torch module over that ABI; finds the
                                library through an $ORIGIN rpath

Both land next to this file so that they travel with the source tree. Run as
``python -m fpscan_amd._build``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
INCLUDE_DIR = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG_DIR, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_LIB = os.path.join(PKG_DIR, "libfpscan_hip.so")
BINDING = os.path.join(PKG_DIR, "_C" + sysconfig.get_config_var("EXT_SUFFIX"))

# gfx950 only. Packed fp32 instructions are disabled for every HIP translation unit.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, label):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; nothing else
    # is expected on a clean build
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        raise RuntimeError(f"{label} failed ({proc.returncode}):\n" + " ".join(cmd) + "\n"
                           + "\n".join(lines[-60:]))
    return "\n".join(lines)


def _atomic_out(path):
    return path + ".tmp%d" % os.getpid()


HIP_SOURCES = ("fpscan_scan.hip", "fpscan_scan_cl.hip", "fpscan_dimwise.hip", "fpscan_probe.hip")


def build_hip_library() -> str:
    srcs = [os.path.join(CSRC, s) for s in HIP_SOURCES]
    tmp = _atomic_out(HIP_LIB)
    _run([HIPCC, *HIP_FLAGS, "-I", INCLUDE_DIR, "-I", CSRC, *srcs, "-o", tmp],
         "hipcc " + " ".join(HIP_SOURCES))
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def _torch_flags():
    import torch
    import torch.utils.cpp_extension as ce

    inc = [f"-I{p}" for p in ce.include_paths()]
    inc.append(f"-I{sysconfig.get_paths()['include']}")
    defs = [
        "-DTORCH_EXTENSION_NAME=_C",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
    ]
    abi = getattr(ce, "_get_pybind11_abi_build_flags", None)
    if abi is not None:
        import warnings

        with warnings.catch_warnings():
            warnings.simplefilter("ignore", DeprecationWarning)
            defs += list(abi())
    libdirs = [f"-L{p}" for p in ce.library_paths()]
    return inc, defs, libdirs


def compile_binding(obj: str) -> str:
    inc, defs, _ = _torch_flags()
    src = os.path.join(CSRC, "binding.cpp")
    cxx = shutil.which("g++") or "g++"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", *defs, *inc,
           f"-I{INCLUDE_DIR}", f"-I{ROCM}/include", "-c", src, "-o", obj]
    _run(cmd, "g++ -c binding.cpp")
    return obj


def link_binding(obj: str) -> str:
    _, _, libdirs = _torch_flags()
    tmp = _atomic_out(BINDING)
    cxx = shutil.which("g++") or "g++"
    cmd = [
        cxx, "-shared", obj, "-o", tmp,
        *libdirs, f"-L{PKG_DIR}", f"-L{ROCM}/lib",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib",
        "-lfpscan_hip", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        "-lamdhip64",
    ]
    _run(cmd, "link _C")
    os.replace(tmp, BINDING)
    return BINDING


def build(verbose: bool = False) -> None:
    """Compiles the HIP library and the binding object in parallel, then links the binding
    against the library."""
    import tempfile

    with tempfile.TemporaryDirectory(prefix="fpscan_build_") as tmpdir:
        obj = os.path.join(tmpdir, "binding.o")
        with concurrent.futures.ThreadPoolExecutor(max_workers=2) as pool:
            lib = pool.submit(build_hip_library)
            cobj = pool.submit(compile_binding, obj)
            lib.result()
            cobj.result()
        link_binding(obj)
    if verbose:
        print(f"built {HIP_LIB}\nbuilt {BINDING}")


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
