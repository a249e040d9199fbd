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
