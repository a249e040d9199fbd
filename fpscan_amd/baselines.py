"""Torch-only reference points for the benchmark CLI (``python -m fpscan_amd.benchmark``).

The names and arguments are those of the reference's eval/baselines.py, so scripts written
against that module run unchanged: ``sequential_scan``, ``parallel_scan_torch`` and
``torch_associative_scan``, each ``f(gates, tokens, reverse=False)`` on (..., seqlen)
tensors, plus ``ASSOCIATIVE_SCAN_AVAILABLE`` and the ``BASELINES`` table. They run on
whatever device their inputs live on and are timing references only: ``fpscan_amd``'s own
entry points never fall back to them.

Each direction is handled by walking or shifting the time axis the other way, without
flipping the tensors.
"""
from __future__ import annotations

import importlib
import inspect
from typing import Callable, Optional, Tuple

import torch

__all__ = [
    "sequential_scan",
    "parallel_scan_torch",
    "torch_associative_scan",
    "ASSOCIATIVE_SCAN_AVAILABLE",
    "BASELINES",
]


def sequential_scan(gates: torch.Tensor, tokens: torch.Tensor,
                    reverse: bool = False) -> torch.Tensor:
    """The recurrence itself, one time index per step (eval/baselines.py:20-37):
    y[t] = gates[t] * y[t-1] + tokens[t] from a zero state, visiting t = L-1 .. 0 instead
    when ``reverse``. Each step is a multiply and an add in the inputs' dtype."""
    length = tokens.shape[-1]
    order = range(length - 1, -1, -1) if reverse else range(length)
    out = torch.empty_like(tokens)
    state = torch.zeros_like(tokens[..., 0])
    for t in order:
        state = gates[..., t] * state + tokens[..., t]
        out[..., t] = state
    return out


def _shifted(t: torch.Tensor, k: int, fill: float, toward_end: bool) -> torch.Tensor:
    """``t`` moved k places along the last axis (toward its end, or toward its start), the
    vacated places holding ``fill``: the element k steps earlier in processing order."""
    pad = t.new_full(t.shape[:-1] + (k,), fill)
    if toward_end:
        return torch.cat((pad, t[..., :-k]), dim=-1)
    return torch.cat((t[..., k:], pad), dim=-1)


def parallel_scan_torch(gates: torch.Tensor, tokens: torch.Tensor,
                        reverse: bool = False) -> torch.Tensor:
    """Hillis-Steele doubling over the affine maps y -> a*y + b (eval/baselines.py:40-61):
    in the pass with distance k every position composes its map with the one k places earlier
    in processing order (the identity (1, 0) where there is none), b with the map's old a:
        b = a * b_earlier + b,  a = a * a_earlier.
    After log2(L) passes, b holds the scan. The same four operations per pass as the
    reference, on whole tensors in their dtype; the reverse direction takes its earlier maps
    from the other side instead of flipping the inputs."""
    a, b = gates, tokens
    length = tokens.shape[-1]
    k = 1
    while k < length:
        a_earlier = _shifted(a, k, 1.0, toward_end=not reverse)
        b_earlier = _shifted(b, k, 0.0, toward_end=not reverse)
        b = a * b_earlier + b
        a = a * a_earlier
        k <<= 1
    return b


# Where torch builds keep associative_scan: the public name first, then the higher-order-op
# module that older builds have it in.
_ASSOCIATIVE_SCAN_HOMES = (("torch", "associative_scan"),
                           ("torch._higher_order_ops.associative_scan", "associative_scan"))


def _locate_associative_scan() -> Optional[Callable]:
    for module_name, attr in _ASSOCIATIVE_SCAN_HOMES:
        try:
            found = getattr(importlib.import_module(module_name), attr, None)
        except ImportError:
            found = None
        if callable(found):
            return found
    return None


def _takes_reverse(fn: Callable) -> bool:
    try:
        return "reverse" in inspect.signature(fn).parameters
    except (TypeError, ValueError):
        return False


_ASSOCIATIVE_SCAN = _locate_associative_scan()
_ASSOCIATIVE_SCAN_REVERSE = _ASSOCIATIVE_SCAN is not None and _takes_reverse(_ASSOCIATIVE_SCAN)
ASSOCIATIVE_SCAN_AVAILABLE = _ASSOCIATIVE_SCAN is not None

Pair = Tuple[torch.Tensor, torch.Tensor]


def _compose(first: Pair, then: Pair) -> Pair:
    """The affine map `first` followed by `then`: y -> a2 * (a1 * y + b1) + b2."""
    return then[0] * first[0], then[0] * first[1] + then[1]


def torch_associative_scan(gates: torch.Tensor, tokens: torch.Tensor,
                           reverse: bool = False) -> torch.Tensor:
    """The scan through torch's own associative_scan with the affine composition
    (eval/baselines.py:80-107). Raises RuntimeError on torch builds without one; on builds
    whose associative_scan has no ``reverse`` argument the time axis is mirrored around it."""
    if _ASSOCIATIVE_SCAN is None:
        raise RuntimeError(f"torch {torch.__version__} has no associative_scan; "
                           "parallel_scan_torch is the torch baseline there")
    if not reverse:
        return _ASSOCIATIVE_SCAN(_compose, (gates, tokens), dim=-1)[1]
    if _ASSOCIATIVE_SCAN_REVERSE:
        return _ASSOCIATIVE_SCAN(_compose, (gates, tokens), dim=-1, reverse=True)[1]
    mirrored = _ASSOCIATIVE_SCAN(_compose, (gates.flip(-1), tokens.flip(-1)), dim=-1)[1]
    return mirrored.flip(-1)


# Labels as in eval/baselines.py's table, which the reference's scripts index by.
BASELINES = dict((
    ("sequential (oracle)", sequential_scan),
    ("torch parallel (hillis-steele)", parallel_scan_torch),
    ("torch.associative_scan", torch_associative_scan),
))
