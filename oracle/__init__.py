"""oracle -- TEST INFRASTRUCTURE ONLY.

The CPU checker for the HIP scan in fpscan_amd/. Only tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py may import it; the product path never does, and has no
CPU fallback of any kind.

What each function restates (saeeddhqan/fpscan, paths relative to the reference root):

  scan_f64              eval/baselines.py:20-37 ``sequential_scan`` -- float64 serial
                        recurrence, zero initial state, reverse by flipping (C: liboracle.so)
  scan_f64_numpy        the same specification, second implementation (numpy, vectorised over
                        rows); exists only to cross-check the C code
  scan_bwd_f64          the gradients of fpscan/ops.py:69-83 ``PScan.backward`` in float64
                        (C: liboracle.so)
  refkernel_f32         the reference CUDA kernel's own fp32 arithmetic, op by op
                        (csrc/full_scan/full_scan.cu:50-177, tiles :207-233); measures the
                        reference's error on the same inputs, never a pass criterion alone
  parallel_scan_torch   eval/baselines.py:40-61 ``parallel_scan_torch`` (Hillis-Steele, same
                        op sequence); the CPU baseline bench.py times
  pscan_backward_composed  fpscan/ops.py:69-83: the backward composed from a scan function
                        (shifted gates, reverse scan, shifted output, product)
  scan_softplus_f64, scan_bwd_softplus_f64
                        scan_f64 / scan_bwd_f64 with gates exp(-softplus(z) * rate[d]) (the
                        fused gate producer; no reference counterpart)
  dimwise_f64           csrc/dimwise/dimwise_scan_final.cu:12-576 -- the contraction scan
                        behind dimwise_forward, in float64 (numpy)
  scan_f64_channel_last, scan_bwd_f64_channel_last
                        the two float64 functions above for (batch, seqlen, dim) tensors
                        scanned along seqlen (README.md:94-99's transpose-in/transpose-out
                        recipe, done on the CPU)

How each is pinned (tests/test_oracle.py): closed forms (g = 1 -> cumsum, g = 0 -> x,
constant g -> geometric series, impulse -> powers of g), brute force from the explicit sum
y[t] = sum_s (prod_{k=s+1..t} g[k]) x[s], exact rational arithmetic (tests/golden), torch
float64 autograd through a serial loop and finite differences (gradcheck) for the backward,
the adjoint identity <go, J v> = <J^T go, v>, and agreement between the two forward
implementations. ``refkernel_f32`` is pinned against exact results on inputs whose every
partial result is exactly representable in fp32. The channel-last pair is pinned against a
direct loop along axis 1, cumsum along axis 1 for g = 1, and float64 autograd through that
loop. The softplus pair is pinned against float64 autograd
through torch's softplus/exp and a serial loop. ``dimwise_f64`` is pinned against a
restatement of the reference's own Python model of
the same computation (scans/contraction_scan.py:98-142, a per-token loop with torch.max for
the selection), against group-sum closed forms, and on ties.

Parity unpinned: dimwise_forward's group selection in fp16/bf16 on the reference's own
input distribution. The reference kernel scans the groups in the native half type
(csrc/dimwise/dimwise_scan_final.cu:12-106), while ``dimwise_f64`` (and the MI355X kernels)
scan them in float64 (fp32), so near-tied group maxima can select a different group. The
half-type tests therefore use inputs whose group maxima are separated by more than the
half type's rounding.
"""
from __future__ import annotations

import ctypes
import os
from typing import Callable, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

__all__ = [
    "scan_f64",
    "scan_f64_numpy",
    "scan_bwd_f64",
    "refkernel_f32",
    "parallel_scan_torch",
    "pscan_backward_composed",
    "normwise_error",
    "to_f64",
]


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        from . import build as _build

        _build.build()
    lib = ctypes.CDLL(_LIB_PATH)
    dp = ctypes.POINTER(ctypes.c_double)
    fp = ctypes.POINTER(ctypes.c_float)
    i64 = ctypes.c_int64
    lib.oracle_scan_f64.argtypes = [dp, dp, dp, i64, i64, ctypes.c_int]
    lib.oracle_scan_f64.restype = None
    lib.oracle_scan_bwd_f64.argtypes = [dp, dp, dp, dp, dp, i64, i64]
    lib.oracle_scan_bwd_f64.restype = None
    lib.oracle_refkernel_f32.argtypes = [fp, fp, fp, i64, i64, ctypes.c_int]
    lib.oracle_refkernel_f32.restype = ctypes.c_int
    _lib = lib
    return lib


def to_f64(a) -> np.ndarray:
    """numpy float64 copy (C-contiguous) of a numpy array or a torch tensor (any device)."""
    try:
        import torch

        if isinstance(a, torch.Tensor):
            return np.ascontiguousarray(a.detach().to("cpu", torch.float64).numpy())
    except ImportError:
        pass
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _rows(a: np.ndarray) -> Tuple[int, int]:
    L = a.shape[-1]
    return (a.size // L if L else 0), L


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def scan_f64(gates, tokens, reverse: bool = False) -> np.ndarray:
    g, x = to_f64(gates), to_f64(tokens)
    assert g.shape == x.shape
    y = np.empty_like(x)
    rows, L = _rows(x)
    if rows and L:
        _load().oracle_scan_f64(_ptr(g, ctypes.c_double), _ptr(x, ctypes.c_double),
                                _ptr(y, ctypes.c_double), rows, L, int(bool(reverse)))
    return y


def scan_f64_numpy(gates, tokens, reverse: bool = False) -> np.ndarray:
    g, x = to_f64(gates), to_f64(tokens)
    if reverse:
        g, x = g[..., ::-1], x[..., ::-1]
    y = np.empty(x.shape, dtype=np.float64)
    state = np.zeros(x.shape[:-1], dtype=np.float64)
    for t in range(x.shape[-1]):
        state = g[..., t] * state + x[..., t]
        y[..., t] = state
    return np.ascontiguousarray(y[..., ::-1]) if reverse else y


def scan_bwd_f64(gates, out, grad_out) -> Tuple[np.ndarray, np.ndarray]:
    """(grad_gates, grad_tokens) in float64, given the forward output ``out``."""
    g, y, go = to_f64(gates), to_f64(out), to_f64(grad_out)
    assert g.shape == y.shape == go.shape
    gg = np.empty_like(g)
    gx = np.empty_like(g)
    rows, L = _rows(g)
    if rows and L:
        _load().oracle_scan_bwd_f64(_ptr(g, ctypes.c_double), _ptr(y, ctypes.c_double),
                                    _ptr(go, ctypes.c_double), _ptr(gg, ctypes.c_double),
                                    _ptr(gx, ctypes.c_double), rows, L)
    return gg, gx


def scan_f64_channel_last(gates, tokens, reverse: bool = False) -> np.ndarray:
    """``scan_f64`` for (batch, seqlen, dim) tensors scanned along seqlen: the same
    recurrences as the (batch, dim, seqlen) transpose, so it transposes, scans and transposes
    back."""
    g = np.swapaxes(to_f64(gates), -1, -2)
    x = np.swapaxes(to_f64(tokens), -1, -2)
    return np.ascontiguousarray(np.swapaxes(scan_f64(g, x, reverse), -1, -2))


def scan_bwd_f64_channel_last(gates, out, grad_out) -> Tuple[np.ndarray, np.ndarray]:
    """``scan_bwd_f64`` for (batch, seqlen, dim) tensors (see ``scan_f64_channel_last``)."""
    sw = lambda a: np.swapaxes(to_f64(a), -1, -2)  # noqa: E731
    gg, gx = scan_bwd_f64(sw(gates), sw(out), sw(grad_out))
    return (np.ascontiguousarray(np.swapaxes(gg, -1, -2)),
            np.ascontiguousarray(np.swapaxes(gx, -1, -2)))


def softplus_gates_f64(z, rate) -> np.ndarray:
    """exp(-softplus(z) * rate[d]) in float64 for (batch, dim, seqlen) z and dim rates."""
    zz = to_f64(z)
    r = to_f64(rate).reshape(1, zz.shape[1], 1)
    return np.exp(-np.logaddexp(0.0, zz) * r)


def scan_softplus_f64(z, rate, tokens, reverse: bool = False) -> np.ndarray:
    """``scan_f64`` with the gates made from z and rate (see ``softplus_gates_f64``)."""
    return scan_f64(softplus_gates_f64(z, rate), tokens, reverse)


def scan_bwd_softplus_f64(z, rate, out, grad_out):
    """(grad_z, grad_rate, grad_tokens) in float64: ``scan_bwd_f64``'s grad_gates carried
    through gate = exp(-softplus(z) * rate) by the chain rule (d softplus / dz = sigmoid)."""
    zz = to_f64(z)
    r = to_f64(rate).reshape(1, zz.shape[1], 1)
    gates = softplus_gates_f64(zz, rate)
    gg, gx = scan_bwd_f64(gates, out, grad_out)
    sig = 0.5 * (1.0 + np.tanh(0.5 * zz))
    grad_z = gg * gates * (-r) * sig
    grad_rate = (gg * gates * (-np.logaddexp(0.0, zz))).sum(axis=(0, 2))
    return grad_z, grad_rate, gx


# (W groups per chunk, P elements per group, C chunks) by seqlen: the reference launcher's
# kernel table, csrc/dimwise/dimwise_scan_final.cu:408-572 (seqlen 32 and others rejected).
DIMWISE_GEOMETRY = {64: (2, 32, 1), 128: (4, 32, 1), 256: (8, 32, 1), 512: (16, 32, 1),
                    1024: (16, 64, 1), 2048: (32, 64, 1), 4096: (32, 128, 1),
                    8192: (32, 128, 2), 16384: (32, 128, 4), 32768: (32, 128, 8),
                    65536: (32, 128, 16)}


def dimwise_f64(Ax, Bx, Bh, Wq, Wk) -> np.ndarray:
    """float64 result of the reference's dimwise_forward (the value it writes into Bx).

    Restates csrc/dimwise/dimwise_scan_final.cu:108-225 (the other kernels are its one-chunk
    cases), per row (b, d): chunks of W groups of P elements; zero-initial-state scans inside
    each group, group 0 starting from the previous chunk's last output (:153-159); v = group
    ends; k = (1+Wk)*Bh[..., :W] (chunk index unused, :133, :189); q = (1+Wq)*v; r[0] = v[0],
    r[g] = s*v[m] + v[g] for 1 <= g <= W-2 with s = k[m]*q[g] the first strict maximum over
    h < g above -1e10 (:195-210; m = 0 where the reference leaves it undefined); outputs
    local + r[g-1] for g >= 1 (:213-219). Ax, Bx: (batch, dim, seqlen); Bh: (batch, dim, W*C);
    Wq, Wk: dim values.
    """
    a, x = to_f64(Ax), to_f64(Bx)
    B, D, L = x.shape
    W, P, C = DIMWISE_GEOMETRY[L]
    k = (1.0 + to_f64(Wk).reshape(1, D, 1)) * to_f64(Bh).reshape(B, D, W * C)[:, :, :W]
    wq1 = 1.0 + to_f64(Wq).reshape(1, D)
    out = np.empty_like(x)
    carry = np.zeros((B, D))
    for c in range(C):
        span = slice(c * W * P, (c + 1) * W * P)
        ac = a[:, :, span].reshape(B, D, W, P).copy()
        xc = x[:, :, span].reshape(B, D, W, P)
        if c == 0:
            ac[:, :, 0, 0] = 1.0  # the row's first gate is never used (:151)
        y = np.zeros((B, D, W))
        y[:, :, 0] = carry
        local = np.empty((B, D, W, P))
        for j in range(P):
            y = ac[..., j] * y + xc[..., j]
            local[..., j] = y
        v = local[..., P - 1]
        r = v.copy()
        for g in range(1, W - 1):
            q = wq1 * v[:, :, g]
            best = np.full((B, D), -1e10)
            m = np.zeros((B, D), dtype=np.int64)
            for h in range(g):
                s = k[:, :, h] * q
                better = s > best
                best = np.where(better, s, best)
                m = np.where(better, h, m)
            vm = np.take_along_axis(v, m[..., None], axis=2)[..., 0]
            r[:, :, g] = best * vm + v[:, :, g]
        outc = local.copy()
        outc[:, :, 1:, :] += r[:, :, :-1, None]
        out[:, :, span] = outc.reshape(B, D, W * P)
        carry = outc[:, :, W - 1, P - 1]
    return out


def refkernel_f32(gates, tokens, reverse: bool = False) -> np.ndarray:
    """fp32 result of the reference kernel's arithmetic (before its final rounding to the
    input dtype: round the result yourself for fp16/bf16)."""
    g = np.ascontiguousarray(to_f64(gates).astype(np.float32))
    x = np.ascontiguousarray(to_f64(tokens).astype(np.float32))
    y = np.empty_like(x)
    rows, L = _rows(x)
    if rows and L:
        rc = _load().oracle_refkernel_f32(_ptr(g, ctypes.c_float), _ptr(x, ctypes.c_float),
                                          _ptr(y, ctypes.c_float), rows, L, int(bool(reverse)))
        if rc == 1:
            raise ValueError(f"the reference kernel rejects seqlen {L}")
        if rc != 0:
            raise MemoryError("oracle_refkernel_f32 could not allocate its work arrays")
    return y


def parallel_scan_torch(gates, tokens, reverse: bool = False):
    """Hillis-Steele scan with torch tensor ops, in the tensors' own dtype and device."""
    import torch.nn.functional as F

    if reverse:
        gates = gates.flip(-1)
        tokens = tokens.flip(-1)
    a, b = gates, tokens
    n = a.shape[-1]
    step = 1
    while step < n:
        a_shift = F.pad(a, (step, 0), value=1.0)[..., :n]
        b_shift = F.pad(b, (step, 0), value=0.0)[..., :n]
        b = a * b_shift + b
        a = a * a_shift
        step *= 2
    return b.flip(-1) if reverse else b


def pscan_backward_composed(gates, out, grad_out, scan: Callable):
    """(grad_gates, grad_tokens) composed from ``scan(gates, tokens, reverse)`` the way the
    reference's PScan.backward does it, in the tensors' dtype."""
    import torch

    grad_out = grad_out.contiguous()
    ones = torch.ones_like(gates[..., :1])
    gates_next = torch.cat([gates[..., 1:], ones], dim=-1).contiguous()
    grad_tokens = scan(gates_next, grad_out, True)
    zeros = torch.zeros_like(out[..., :1])
    out_prev = torch.cat([zeros, out[..., :-1]], dim=-1)
    return out_prev * grad_tokens, grad_tokens


def normwise_error(y, ref) -> float:
    """max |y - ref| / max |ref| over the whole tensor, in float64 (0 when both are 0)."""
    a, b = to_f64(y), to_f64(ref)
    denom = float(np.max(np.abs(b))) if b.size else 0.0
    num = float(np.max(np.abs(a - b))) if b.size else 0.0
    if denom == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / denom
