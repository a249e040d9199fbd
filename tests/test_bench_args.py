"""bench.py's argument handling: the refusals that come before any device is touched, so they
run here without a GPU."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*argv):
    env = dict(os.environ, WORLD_SIZE="1")
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *argv], cwd=ROOT,
                          env=env, capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("argv, message", [
    (["--workload", "rows"], "--workload rows needs --shape"),
    (["--workload", "rows", "--shape", "8,1024"], "three positive integers"),
    (["--workload", "dw", "--shape", "8,x,65536"], "three positive integers"),
    (["--workload", "rows", "--shape", "0,1024,65536"], "three positive integers"),
])
def test_bad_shapes_are_refused_before_any_device_check(argv, message):
    r = _bench(*argv)
    assert r.returncode == 2
    assert message in r.stderr and r.stdout == ""
