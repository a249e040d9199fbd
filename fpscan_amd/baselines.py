"""Baselines that fpscan_amd's benchmark compares the HIP scan against, with the API of the
reference's eval/baselines.py (same names and arguments), all on torch tensor ops:

* ``sequential_scan``       eval/baselines.py:20-37 -- one step per time index
* ``parallel_scan_torch``   eval/baselines.py:40-61 -- Hillis-Steele doubling, log2(L) passes,
                            the pair (a, b) updated with b taking the old a
* ``torch_associative_scan`` eval/baselines.py:64-107 -- torch's associative_scan with the
                            affine combine, where this torch build has one

They are reference points for timing, never a fallback: ``fpscan_amd.scan_forward`` only runs
the HIP kernels.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch
import torch.nn.functional as F

__all__ = [
    "sequential_scan",
    "parallel_scan_torch",
    "torch_associative_scan",
    "ASSOCIATIVE_SCAN_AVAILABLE",
    "BASELINES",
]


def _in_order(gates: torch.Tensor, tokens: torch.Tensor, reverse: bool):
    return (gates.flip(-1), tokens.flip(-1)) if reverse else (gates, tokens)


def sequential_scan(gates: torch.Tensor, tokens: torch.Tensor,
                    reverse: bool = False) -> torch.Tensor:
    """y[t] = gates[t] * y[t-1] + tokens[t] (reverse: from the end), one time index at a time."""
    g, x = _in_order(gates, tokens, reverse)
    out = torch.empty_like(x)
    state = torch.zeros_like(x[..., 0])
    for t in range(x.shape[-1]):
        state = g[..., t] * state + x[..., t]
        out[..., t] = state
    return out.flip(-1) if reverse else out


def parallel_scan_torch(gates: torch.Tensor, tokens: torch.Tensor,
                        reverse: bool = False) -> torch.Tensor:
    """Hillis-Steele scan of the affine maps: after the pass with shift s every position holds
    the composition of the last 2s maps; positions before the start see the identity (1, 0)."""
    a, b = _in_order(gates, tokens, reverse)
    n = a.shape[-1]
    shift = 1
    while shift < n:
        a_before = F.pad(a, (shift, 0), value=1.0)[..., :n]
        b_before = F.pad(b, (shift, 0), value=0.0)[..., :n]
        b = a * b_before + b
        a = a * a_before
        shift *= 2
    return b.flip(-1) if reverse else b


def _find_associative_scan() -> Optional[Callable]:
    found = getattr(torch, "associative_scan", None)
    if found is not None:
        return found
    try:
        from torch._higher_order_ops.associative_scan import associative_scan
    except Exception:
        return None
    return associative_scan


_ASSOCIATIVE_SCAN = _find_associative_scan()
ASSOCIATIVE_SCAN_AVAILABLE = _ASSOCIATIVE_SCAN is not None


def _affine_combine(earlier, later):
    a0, b0 = earlier
    a1, b1 = later
    return a1 * a0, a1 * b0 + b1


def torch_associative_scan(gates: torch.Tensor, tokens: torch.Tensor,
                           reverse: bool = False) -> torch.Tensor:
    """The scan through torch's associative_scan (raises RuntimeError where torch has none)."""
    if _ASSOCIATIVE_SCAN is None:
        raise RuntimeError(f"torch.associative_scan is not available in torch {torch.__version__};"
                           " use parallel_scan_torch")
    try:
        return _ASSOCIATIVE_SCAN(_affine_combine, (gates, tokens), dim=-1, reverse=reverse)[1]
    except TypeError:  # builds whose associative_scan has no `reverse`
        g, x = _in_order(gates, tokens, reverse)
        out = _ASSOCIATIVE_SCAN(_affine_combine, (g, x), dim=-1)[1]
        return out.flip(-1) if reverse else out


BASELINES = {
    "sequential (oracle)": sequential_scan,
    "torch parallel (hillis-steele)": parallel_scan_torch,
    "torch.associative_scan": torch_associative_scan,
}
