"""Inputs, tolerances and comparisons shared by the GPU parity tests."""
import numpy as np
import torch

import oracle

DEVICE = "cuda"
ALL_SEQLENS = [32, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768, 65536]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]

REF_TOL = {  # reference tests/test_fpscan.py:18-22 (elementwise assert_close)
    torch.float32: dict(atol=2e-3, rtol=2e-3),
    torch.float16: dict(atol=3e-2, rtol=3e-2),
    torch.bfloat16: dict(atol=6e-2, rtol=6e-2),
}
NORM_TOL = {torch.float32: 1e-5, torch.float16: 5e-3, torch.bfloat16: 2e-2}  # north star


def make_inputs(batch, dim, seqlen, dtype, seed=0):
    """test_fpscan.py:25-29 distributions, drawn on a seeded CPU generator (portable)."""
    gen = torch.Generator().manual_seed(seed)
    gates = 0.99 + 0.01 * torch.rand(batch, dim, seqlen, generator=gen)
    tokens = torch.randn(batch, dim, seqlen, generator=gen) / seqlen
    return gates.to(dtype).contiguous(), tokens.to(dtype).contiguous()


def check(got, ref, dtype, what=""):
    err = oracle.normwise_error(got, ref)
    assert err <= NORM_TOL[dtype], f"{what}: normwise error {err:.3e} > {NORM_TOL[dtype]}"
    torch.testing.assert_close(got.detach().double().cpu(), torch.from_numpy(np.asarray(ref)),
                               **REF_TOL[dtype], msg=lambda m: f"{what}: {m}")
    return err


def bits_equal(a, b):
    return torch.equal(a.contiguous().view(torch.int16 if a.element_size() == 2 else torch.int32),
                       b.contiguous().view(torch.int16 if b.element_size() == 2 else torch.int32))


# ------------------------------------------------------------------ narrowing (rounding) inputs
# Offsets that put the running sums where fp16 / bf16 must round: bf16 keeps 8 significant
# bits, so integers from 256 up are spaced 2, 4, 8 ...; fp16 keeps 11, spaced 2 from 2048.
# Both offsets are exact in their type (1000 = 0b1111101000, 3000 = 0b101110111000).
ROUNDING_OFFSET = {torch.bfloat16: 1000.0, torch.float16: 3000.0, torch.float32: 1000.0}


def rounding_inputs(shape, dtype, axis=-1, reverse=False, step=7, seed=0):
    """Gates 1 and integer tokens in [-step, step], with the element processed first set to
    ROUNDING_OFFSET[dtype]: every partial result of any combine order is an integer below
    2^24, exact in fp32, while most final values need more significant bits than fp16/bf16
    hold and many sit exactly halfway between two neighbours. A kernel's stored outputs are
    then the exact sums rounded once, so the comparison sees the narrowing rule itself."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randint(-step, step + 1, shape, generator=gen).double()
    idx = [slice(None)] * len(shape)
    idx[axis] = -1 if reverse else 0
    x[tuple(idx)] = ROUNDING_OFFSET[dtype]
    return torch.ones(shape, dtype=dtype), x.to(dtype)


def narrowed(exact, dtype):
    """Exact (float64, fp32-representable) values rounded to nearest-even in ``dtype`` on the
    CPU -- the reference's __float2half / __float2bfloat16 (csrc/full_scan/conversion.h:7-13)."""
    t = torch.as_tensor(np.asarray(exact))
    f32 = t.float()
    assert torch.equal(f32.double(), t.double()), "expected values must be exact in fp32"
    return f32.to(dtype)


def truncated(exact, dtype):
    """The same values rounded toward zero: what a truncating narrowing would store."""
    t = torch.as_tensor(np.asarray(exact)).double()
    r = t.float().to(dtype)
    bits = r.view(torch.int16 if r.element_size() == 2 else torch.int32).clone()
    over = r.double().abs() > t.abs()  # rounded away from zero: step one ulp back
    bits[over] -= 1
    return bits.view(dtype)


def rounding_counts(exact, dtype):
    """(inexact, ties): how many values do not fit ``dtype`` and how many of those sit exactly
    halfway between two neighbours (where round-to-nearest-even is the only rule that matters)."""
    t = torch.as_tensor(np.asarray(exact)).double()
    lo = truncated(t, dtype).double()
    inexact = lo != t
    bits = truncated(t, dtype).view(torch.int16 if torch.empty((), dtype=dtype).element_size() == 2
                                    else torch.int32) + 1
    hi = bits.view(dtype).double()  # one ulp further from zero
    ties = inexact & ((t - lo).abs() == (hi - t).abs())
    return int(inexact.sum()), int(ties.sum())
