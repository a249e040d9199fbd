"""Python API of the MI355X scan: ``scan_forward``, ``PScan`` and ``pscan``.

Drop-in for ``fpscan/ops.py`` of saeeddhqan/fpscan:

* ``_load_extension`` mirrors fpscan/ops.py:20-44 (first importable candidate that exposes
  ``fullscan_forward``, ImportError listing every failure otherwise). There is no fallback:
  without the built HIP extension every entry point raises.
* ``scan_forward`` mirrors fpscan/ops.py:47-58 (caller-provided or freshly allocated ``out``,
  returned after the call).
* ``PScan.forward`` mirrors fpscan/ops.py:63-67 (saves ``(gates, out)``).
* ``PScan.backward`` replaces fpscan/ops.py:69-83 (shifted-gate copy, reverse scan,
  shifted-output copy, product: 7 ATen launches and one scan) with one fused HIP kernel that
  reads gates, out and grad_out once and writes both gradients.
* ``pscan`` mirrors fpscan/ops.py:86-87; the autograd function it applies is the C++ twin of
  ``PScan`` in the extension (same saved tensors, same kernels), which spares the engine a
  Python call in the forward and in the backward. ``PScan.apply`` keeps working.
"""
from __future__ import annotations

import importlib
from typing import Optional, Tuple

import torch

__all__ = ["pscan", "scan_forward", "scan_backward", "PScan", "pscan_channel_last",
           "scan_forward_channel_last", "scan_backward_channel_last", "PScanChannelLast",
           "pscan_softplus", "scan_forward_softplus", "scan_backward_softplus", "PScanSoftplus"]

_EXT_CANDIDATES = ("fpscan_amd._C",)
_ext = None


def _load_extension():
    global _ext
    if _ext is not None:
        return _ext

    errors = []
    for name in _EXT_CANDIDATES:
        try:
            module = importlib.import_module(name)
        except Exception as exc:  # not built / wrong arch / missing ROCm runtime
            errors.append(f"  {name}: {exc}")
            continue
        if hasattr(module, "fullscan_forward"):
            _ext = module
            return _ext
        errors.append(f"  {name}: imported but has no 'fullscan_forward'")

    raise ImportError(
        "Could not import the fpscan HIP extension. Build it first "
        "(`python -c 'import __graft_entry__ as g; g.build()'` from the repository root, "
        "or `python -m fpscan_amd._build`). Tried:\n" + "\n".join(errors)
    )


def scan_forward(
    gates: torch.Tensor,
    tokens: torch.Tensor,
    reverse: bool = False,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """y[t] = gates[t]*y[t-1] + tokens[t] along the last axis (reverse: y[t+1]), y = 0 before
    the first element. (batch, dim, seqlen) contiguous fp32/fp16/bf16 on the GPU, seqlen a
    power of two in [32, 65536]; fp32 accumulation. Writes into ``out`` when given."""
    ext = _load_extension()
    if out is None:
        out = torch.empty_like(tokens)
    ext.fullscan_forward(gates, tokens, out, reverse)
    return out


def scan_backward(
    gates: torch.Tensor,
    out: torch.Tensor,
    grad_out: torch.Tensor,
    grad_gates: Optional[torch.Tensor] = None,
    grad_tokens: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gradients of the forward scan given its output ``out``:
    grad_tokens[t] = grad_out[t] + gates[t+1]*grad_tokens[t+1] (gates[L] = 1) and
    grad_gates[t] = grad_tokens[t]*out[t-1] (out[-1] = 0). Returns (grad_gates, grad_tokens).
    """
    ext = _load_extension()
    if grad_gates is None:
        grad_gates = torch.empty_like(gates)
    if grad_tokens is None:
        grad_tokens = torch.empty_like(gates)
    ext.fullscan_backward(gates, out, grad_out, grad_gates, grad_tokens)
    return grad_gates, grad_tokens


class PScan(torch.autograd.Function):

    @staticmethod
    def forward(ctx, gates: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
        out = scan_forward(gates, tokens)
        ctx.save_for_backward(gates, out)
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        gates, out = ctx.saved_tensors
        grad_output = grad_output.contiguous()
        grad_gates, grad_tokens = scan_backward(gates, out, grad_output)
        return grad_gates, grad_tokens


def pscan(gates: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Differentiable ``scan_forward(gates, tokens)``: the computation of ``PScan.apply``
    (fpscan/ops.py:86-87), run by the extension's C++ autograd function so that neither the
    forward nor the backward makes a Python call (the host time of a short step)."""
    return _load_extension().pscan(gates, tokens)


# ---------------------------------------------------------------------------------------
# Channel-last layout: (batch, seqlen, dim), scanned along seqlen. No reference counterpart;
# the reference's README.md:94-99 transposes in and out around pscan instead, which this
# path makes unnecessary (same results, no copies).
# ---------------------------------------------------------------------------------------
def scan_forward_channel_last(
    gates: torch.Tensor,
    tokens: torch.Tensor,
    reverse: bool = False,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """y[:, t] = gates[:, t]*y[:, t-1] + tokens[:, t] for (batch, seqlen, dim) contiguous
    fp32/fp16/bf16 tensors (reverse: y[:, t+1]); any seqlen >= 1, dim a multiple of
    16/itemsize. Equal to ``scan_forward(g.mT.contiguous(), x.mT.contiguous()).mT`` up to fp32
    rounding order."""
    ext = _load_extension()
    if out is None:
        out = torch.empty_like(tokens)
    ext.fullscan_forward_cl(gates, tokens, out, reverse)
    return out


def scan_backward_channel_last(
    gates: torch.Tensor,
    out: torch.Tensor,
    grad_out: torch.Tensor,
    grad_gates: Optional[torch.Tensor] = None,
    grad_tokens: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gradients of ``scan_forward_channel_last`` given its output: grad_tokens[:, t] =
    grad_out[:, t] + gates[:, t+1]*grad_tokens[:, t+1] and grad_gates[:, t] =
    grad_tokens[:, t]*out[:, t-1]. Returns (grad_gates, grad_tokens)."""
    ext = _load_extension()
    if grad_gates is None:
        grad_gates = torch.empty_like(gates)
    if grad_tokens is None:
        grad_tokens = torch.empty_like(gates)
    ext.fullscan_backward_cl(gates, out, grad_out, grad_gates, grad_tokens)
    return grad_gates, grad_tokens


class PScanChannelLast(torch.autograd.Function):

    @staticmethod
    def forward(ctx, gates: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
        out = scan_forward_channel_last(gates, tokens)
        ctx.save_for_backward(gates, out)
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        gates, out = ctx.saved_tensors
        grad_output = grad_output.contiguous()
        grad_gates, grad_tokens = scan_backward_channel_last(gates, out, grad_output)
        return grad_gates, grad_tokens


def pscan_channel_last(gates: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Differentiable scan of (batch, seqlen, dim) tensors along seqlen."""
    return PScanChannelLast.apply(gates, tokens)


# ---------------------------------------------------------------------------------------
# Fused gate producer: gates = exp(-softplus(z) * rate[d]) (a Mamba-style decay:
# delta = softplus(z), A = -rate) computed inside the scan, so the gates tensor is never
# written or read. No reference counterpart; it replaces "compute gates, then pscan".
# ---------------------------------------------------------------------------------------
def scan_forward_softplus(
    z: torch.Tensor,
    rate: torch.Tensor,
    tokens: torch.Tensor,
    reverse: bool = False,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``scan_forward(torch.exp(-softplus(z) * rate[:, None]), tokens, reverse)`` without the
    gates tensor. z, tokens: (batch, dim, seqlen) contiguous of one dtype; rate: float32,
    one value per dim."""
    ext = _load_extension()
    if out is None:
        out = torch.empty_like(tokens)
    ext.fullscan_forward_softplus(z, rate, tokens, out, reverse)
    return out


def scan_backward_softplus(
    z: torch.Tensor,
    rate: torch.Tensor,
    out: torch.Tensor,
    grad_out: torch.Tensor,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(grad_z, grad_rate, grad_tokens) of ``scan_forward_softplus`` (forward direction)
    given its output. grad_rate is float32 with rate's shape: the kernel writes one partial
    sum per (batch, dim) row and the batch is summed here."""
    ext = _load_extension()
    grad_z = torch.empty_like(z)
    grad_tokens = torch.empty_like(z)
    B, D = z.shape[0], z.shape[1]
    rows = torch.empty(B * D, dtype=torch.float32, device=z.device)
    ext.fullscan_backward_softplus(z, rate, out, grad_out, grad_z, grad_tokens, rows)
    return grad_z, rows.view(B, D).sum(0).view(rate.shape), grad_tokens


class PScanSoftplus(torch.autograd.Function):

    @staticmethod
    def forward(ctx, z: torch.Tensor, rate: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
        out = scan_forward_softplus(z, rate, tokens)
        ctx.save_for_backward(z, rate, out)
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        z, rate, out = ctx.saved_tensors
        grad_z, grad_rate, grad_tokens = scan_backward_softplus(z, rate, out,
                                                                grad_output.contiguous())
        return grad_z, grad_rate, grad_tokens


def pscan_softplus(z: torch.Tensor, rate: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Differentiable ``pscan(torch.exp(-softplus(z) * rate[:, None]), tokens)`` with the
    gates computed inside the kernels (forward and backward)."""
    return PScanSoftplus.apply(z, rate, tokens)


# ---------------------------------------------------------------------------------------
# Contraction scan: the reference module's dimwise_forward (csrc/main.cpp:10), used by its
# scans/contraction_scan.py. In place into Bx, returns None, no backward (as the reference).
# ---------------------------------------------------------------------------------------
def dimwise_forward(Ax: torch.Tensor, Bx: torch.Tensor, Bh: torch.Tensor, Wq: torch.Tensor,
                    Wk: torch.Tensor) -> None:
    """Group scans of (batch, dim, seqlen) rows mixed across groups by a first-maximum
    selection over (1+Wk)*Bh and (1+Wq)*v, written into Bx. Bh is (batch, dim,
    dimwise_groups(seqlen)); Wq and Wk have one entry per dim."""
    _load_extension().dimwise_forward(Ax, Bx, Bh, Wq, Wk)


def dimwise_groups(seqlen: int) -> int:
    """Bh entries per row that dimwise_forward expects for ``seqlen`` (0: unsupported)."""
    return int(_load_extension().dimwise_groups(int(seqlen)))


_DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def dimwise_workspace_bytes(batch: int, dim: int, seqlen: int, dtype: torch.dtype) -> int:
    """Workspace dimwise_forward allocates for this problem: nonzero exactly when it takes the
    tiled path (which depends on ``set_tiling``), 0 when it takes the row kernel."""
    return int(_load_extension().dimwise_workspace_bytes(int(batch), int(dim), int(seqlen),
                                                         _DTYPE_CODE[dtype]))


def set_launch_override(waves_per_row: int = 0, ring_depth: int = 0) -> None:
    """Tuning hook: force the number of waves per row and the per-wave ring depth of the
    long-row kernels (0 restores the built-in choice). Process-wide."""
    _load_extension().set_launch_override(int(waves_per_row), int(ring_depth))


def lookback_overruns(device=None) -> int:
    """Look-back waits of the tiled kernels that gave up on ``device`` (default: the current
    one) since the library was loaded; 0 in a correct run. Waits for the device first. A wait
    gives up only if an earlier tile stalls for tens of milliseconds; the affected outputs
    are then NaN, and this count says so."""
    dev = torch.cuda.current_device() if device is None else torch.device(device).index
    return int(_load_extension().lookback_overruns(int(dev if dev is not None else 0)))


def check_lookback(device=None) -> None:
    """Raises RuntimeError if any look-back wait has given up on ``device`` (whose outputs
    then hold NaN). It synchronises the whole device first (hipDeviceSynchronize) and then
    copies one counter back, so it drains all queued work: call it at a point where the
    caller synchronises anyway, such as the end of a training step or of an epoch, not
    after every scan."""
    n = lookback_overruns(device)
    if n:
        raise RuntimeError(f"fpscan: {n} look-back wait(s) of the tiled scan gave up on this "
                           "device; the outputs of the affected tiles are NaN")


def set_lookback_test_hook(unpublished_tile: int = -1, spin_limit: int = 0) -> None:
    """Test hook (process-wide): the tiled kernels never publish tile ``unpublished_tile``'s
    map, and a look-back wait gives up after ``spin_limit`` polls (0: the default). The
    defaults restore normal operation."""
    _load_extension().set_lookback_test_hook(int(unpublished_tile), int(spin_limit))


def set_tiling(mode: int = 0) -> None:
    """Path selection (process-wide) for long rows, channel-last scans and dimwise_forward:
    0 automatic, 1 no tiled look-back (rows streamed; channel-last one pass per strip or
    segments; dimwise's row kernel), 2 tiled (persistent grid with look-back) whenever the
    shape allows."""
    _load_extension().set_tiling(int(mode))
