"""Shared test setup.

* Puts the repository root on sys.path (as the reference's conftest.py:5 does) so that
  ``fpscan_amd``, ``oracle`` and ``bench`` import from the checkout.
* Registers the ``gpu`` marker: tests that launch HIP kernels. The CPU suite is
  ``pytest -m "not gpu"``; the GPU suite is ``pytest -m gpu`` on an MI355X.
* Builds oracle/liboracle.so (gcc) when it is missing; the HIP extension is never built
  here -- tests load what ``__graft_entry__.build()`` produced.
"""
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "known_answers.json")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: launches HIP kernels; needs an MI355X (gfx950)")


@pytest.fixture(scope="session")
def known_answers():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()
