"""Builds oracle/liboracle.so from oracle/scan_oracle.c (gcc, OpenMP).

TEST INFRASTRUCTURE ONLY: the library is the checker the tests, the smoke check and the
cpu_baseline leg of bench.py compare against; the product never loads it.

The reference's own kernel (csrc/full_scan/full_scan.cu) is CUDA and cannot be compiled in
this image (no nvcc; hipify is not a build route here), so there is no oracle/_ref build:
oracle/scan_oracle.c restates it instead (oracle_refkernel_f32).
"""
from __future__ import annotations

import os
import shutil
import subprocess

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(ORACLE_DIR, "scan_oracle.c")
LIBRARY = os.path.join(ORACLE_DIR, "liboracle.so")


def build(verbose: bool = False) -> str:
    cc = shutil.which("gcc") or "cc"
    tmp = LIBRARY + ".tmp%d" % os.getpid()
    # -ffp-contract=off: only the explicit fmaf() calls fuse, exactly as written
    cmd = [cc, "-O2", "-fopenmp", "-ffp-contract=off", "-fPIC", "-shared", "-std=c11",
           SOURCE, "-o", tmp, "-lm"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + " ".join(cmd) + "\n" + proc.stdout)
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
