"""MI355X-native first-order linear-recurrence scan (drop-in for saeeddhqan/fpscan).

Same public names as fpscan/__init__.py:1-3 (``pscan``, ``scan_forward``, ``PScan``), plus
``scan_backward`` (the fused backward, exposed directly).
"""
from .ops import PScan, pscan, scan_backward, scan_forward

__all__ = ["pscan", "scan_forward", "scan_backward", "PScan"]
__version__ = "0.1.2"
