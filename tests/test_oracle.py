"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernels.

Every oracle function is checked against something it does not share code or formula with:
closed forms, the explicit-sum solution of the recurrence, exact rational known answers
(tests/golden), torch float64 autograd and finite differences, and the adjoint identity.
A plausible mistake -- a dropped gate, an off-by-one shift, reverse running the wrong way, a
swapped operand -- fails at least one of these.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle

RNG = np.random.default_rng(1234)


def rand_inputs(rows, L, lo=0.5, hi=1.0, seed=None):
    rng = np.random.default_rng(seed) if seed is not None else RNG
    g = rng.uniform(lo, hi, size=(rows, L))
    x = rng.standard_normal(size=(rows, L))
    return g, x


# ---------------------------------------------------------------- forward / reverse
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("L", [1, 2, 7, 32, 100])
def test_c_and_numpy_restatements_agree(L, reverse):
    g, x = rand_inputs(5, L)
    a = oracle.scan_f64(g, x, reverse)
    b = oracle.scan_f64_numpy(g, x, reverse)
    np.testing.assert_array_equal(a, b)  # same operations in the same order


@pytest.mark.parametrize("L", [1, 3, 6, 9])
def test_forward_matches_explicit_sum(L):
    """y[t] = sum_{s<=t} (prod_{k=s+1..t} g[k]) x[s]: the closed-form solution."""
    g, x = rand_inputs(3, L, lo=-1.5, hi=1.5)
    want = np.zeros_like(x)
    for t in range(L):
        for s in range(t + 1):
            want[:, t] += np.prod(g[:, s + 1:t + 1], axis=1) * x[:, s]
    np.testing.assert_allclose(oracle.scan_f64(g, x), want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("L", [1, 3, 6, 9])
def test_reverse_matches_explicit_sum(L):
    """reverse: y[t] = sum_{s>=t} (prod_{k=t..s-1} g[k]) x[s]."""
    g, x = rand_inputs(3, L, lo=-1.5, hi=1.5)
    want = np.zeros_like(x)
    for t in range(L):
        for s in range(t, L):
            want[:, t] += np.prod(g[:, t:s], axis=1) * x[:, s]
    np.testing.assert_allclose(oracle.scan_f64(g, x, True), want, rtol=1e-12, atol=1e-12)


def test_gate_one_is_cumsum():
    x = RNG.integers(-5, 6, size=(4, 64)).astype(np.float64)
    np.testing.assert_array_equal(oracle.scan_f64(np.ones_like(x), x), np.cumsum(x, axis=1))
    np.testing.assert_array_equal(oracle.scan_f64(np.ones_like(x), x, True),
                                  np.cumsum(x[:, ::-1], axis=1)[:, ::-1])


def test_gate_zero_is_identity():
    x = RNG.standard_normal((4, 64))
    np.testing.assert_array_equal(oracle.scan_f64(np.zeros_like(x), x), x)
    np.testing.assert_array_equal(oracle.scan_f64(np.zeros_like(x), x, True), x)


@pytest.mark.parametrize("gval", [0.5, 0.9, 0.99998, -0.7])
def test_constant_gate_geometric_series(gval):
    L = 200
    g = np.full((1, L), gval)
    t = np.arange(L)
    want = (1.0 - gval ** (t + 1)) / (1.0 - gval)
    np.testing.assert_allclose(oracle.scan_f64(g, np.ones((1, L)))[0], want, rtol=1e-11)


def test_impulse_response_is_power_of_gate():
    L, s, gval = 50, 7, 0.8
    x = np.zeros((1, L))
    x[0, s] = 1.0
    y = oracle.scan_f64(np.full((1, L), gval), x)[0]
    want = np.where(np.arange(L) >= s, gval ** np.clip(np.arange(L) - s, 0, None), 0.0)
    np.testing.assert_allclose(y, want, rtol=1e-13, atol=0)


def test_reverse_is_flipped_forward_and_rows_are_independent():
    g, x = rand_inputs(6, 33)
    np.testing.assert_array_equal(oracle.scan_f64(g, x, True),
                                  oracle.scan_f64(g[:, ::-1], x[:, ::-1])[:, ::-1])
    # one row alone gives the same answer as inside the batch (no cross-row leakage)
    np.testing.assert_array_equal(oracle.scan_f64(g[3:4], x[3:4]), oracle.scan_f64(g, x)[3:4])


def test_linear_in_tokens():
    g, x1 = rand_inputs(3, 40)
    _, x2 = rand_inputs(3, 40)
    lhs = oracle.scan_f64(g, 2.5 * x1 - 0.5 * x2)
    rhs = 2.5 * oracle.scan_f64(g, x1) - 0.5 * oracle.scan_f64(g, x2)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-12, atol=1e-12)


def test_first_gate_only_matters_through_zero_state():
    g, x = rand_inputs(2, 16)
    g2 = g.copy()
    g2[:, 0] = 123.0
    np.testing.assert_array_equal(oracle.scan_f64(g, x), oracle.scan_f64(g2, x))


# ---------------------------------------------------------------- known answers (exact)
def _frac_rows(rows):
    return np.array([[float(Fraction(v)) for v in r] for r in rows], dtype=np.float64)


def test_known_answers(known_answers):
    for case in known_answers:
        g, x = _frac_rows(case["gates"]), _frac_rows(case["tokens"])
        exact_ints = not case["name"].startswith("dyadic")
        for key, rev in (("forward", False), ("reverse", True)):
            want = np.array(case[key])
            got = oracle.scan_f64(g, x, rev)
            if exact_ints:
                np.testing.assert_array_equal(got, want, err_msg=case["name"])
            else:
                np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-15, err_msg=case["name"])
        if "grad_out" in case:
            go = _frac_rows(case["grad_out"])
            gg, gx = oracle.scan_bwd_f64(g, oracle.scan_f64(g, x), go)
            np.testing.assert_allclose(gx, np.array(case["grad_tokens"]), rtol=1e-13, atol=1e-15)
            np.testing.assert_allclose(gg, np.array(case["grad_gates"]), rtol=1e-13, atol=1e-15)


def test_all_ones_known_answer(known_answers):
    """scans/full_scan.py:54-82 of the reference: all-ones inputs give y[t] = t + 1."""
    case = next(c for c in known_answers if c["name"] == "all_ones")
    np.testing.assert_array_equal(np.array(case["forward"])[0], np.arange(1, 33))


# ---------------------------------------------------------------- backward
def _torch_serial_scan(g, x):
    out = []
    acc = torch.zeros_like(x[..., 0])
    for t in range(x.shape[-1]):
        acc = g[..., t] * acc + x[..., t]
        out.append(acc)
    return torch.stack(out, dim=-1)


@pytest.mark.parametrize("L", [1, 2, 5, 32])
def test_backward_matches_torch_autograd(L):
    g, x = rand_inputs(3, L, lo=-1.2, hi=1.2)
    go = RNG.standard_normal((3, L))
    gt = torch.tensor(g, requires_grad=True)
    xt = torch.tensor(x, requires_grad=True)
    (_torch_serial_scan(gt, xt) * torch.tensor(go)).sum().backward()
    gg, gx = oracle.scan_bwd_f64(g, oracle.scan_f64(g, x), go)
    np.testing.assert_allclose(gx, xt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gg, gt.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_backward_gradcheck_finite_differences():
    """torch.autograd.gradcheck (finite differences) on a Function built from the oracle."""

    class OracleScan(torch.autograd.Function):
        @staticmethod
        def forward(ctx, g, x):
            y = torch.from_numpy(oracle.scan_f64(g.numpy(), x.numpy()))
            ctx.save_for_backward(g, y)
            return y

        @staticmethod
        def backward(ctx, go):
            g, y = ctx.saved_tensors
            gg, gx = oracle.scan_bwd_f64(g.numpy(), y.numpy(), go.numpy())
            return torch.from_numpy(gg), torch.from_numpy(gx)

    g, x = rand_inputs(2, 7, lo=-1.0, hi=1.0)
    gt = torch.tensor(g, requires_grad=True)
    xt = torch.tensor(x, requires_grad=True)
    assert torch.autograd.gradcheck(OracleScan.apply, (gt, xt), eps=1e-6, atol=1e-7)


def test_backward_adjoint_identity():
    """<go, J v> = <J^T go, v> for the token Jacobian J = d y / d x (linear in x)."""
    g, _ = rand_inputs(4, 50)
    v = RNG.standard_normal((4, 50))
    go = RNG.standard_normal((4, 50))
    jv = oracle.scan_f64(g, v)  # y is linear in x, so J v = scan(g, v)
    _, jt_go = oracle.scan_bwd_f64(g, np.zeros_like(g), go)
    assert abs(np.sum(go * jv) - np.sum(jt_go * v)) < 1e-10 * np.sum(np.abs(go * jv))


def test_backward_first_grad_gate_is_zero_and_last_grad_token_is_grad_out():
    g, x = rand_inputs(3, 20)
    go = RNG.standard_normal((3, 20))
    gg, gx = oracle.scan_bwd_f64(g, oracle.scan_f64(g, x), go)
    np.testing.assert_array_equal(gg[:, 0], 0.0)
    np.testing.assert_array_equal(gx[:, -1], go[:, -1])


# ---------------------------------------------------------------- baselines and the
# reference-kernel emulation
@pytest.mark.parametrize("L", [1, 2, 3, 64, 100])
@pytest.mark.parametrize("reverse", [False, True])
def test_hillis_steele_matches_oracle(L, reverse):
    g, x = rand_inputs(4, L)
    got = oracle.parallel_scan_torch(torch.tensor(g), torch.tensor(x), reverse).numpy()
    np.testing.assert_allclose(got, oracle.scan_f64(g, x, reverse), rtol=1e-12, atol=1e-12)


def test_composed_backward_matches_oracle_backward():
    g, x = rand_inputs(3, 48)
    go = RNG.standard_normal((3, 48))
    y = oracle.scan_f64(g, x)

    def scan(a, b, reverse):
        return torch.from_numpy(oracle.scan_f64(a.numpy(), b.numpy(), reverse))

    gg, gx = oracle.pscan_backward_composed(torch.tensor(g), torch.tensor(y),
                                            torch.tensor(go), scan)
    want_gg, want_gx = oracle.scan_bwd_f64(g, y, go)
    np.testing.assert_allclose(gx.numpy(), want_gx, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(gg.numpy(), want_gg, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("L", [32, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 65536])
@pytest.mark.parametrize("reverse", [False, True])
def test_refkernel_exact_on_representable_inputs(L, reverse):
    """Gates in {0, 1} and small integer tokens: every partial result is an exact fp32
    integer, so the emulated reference kernel must equal the exact scan in any order."""
    rng = np.random.default_rng(L)
    g = (rng.integers(0, 16, size=(2, L)) > 0).astype(np.float64)
    x = rng.integers(-3, 4, size=(2, L)).astype(np.float64)
    np.testing.assert_array_equal(oracle.refkernel_f32(g, x, reverse),
                                  oracle.scan_f64(g, x, reverse))


@pytest.mark.parametrize("L", [32, 64, 1024, 8192, 65536])
@pytest.mark.parametrize("reverse", [False, True])
def test_refkernel_close_to_oracle(L, reverse):
    rng = np.random.default_rng(L + 7)
    g = (0.99 + 0.01 * rng.random((2, L))).astype(np.float32)
    x = (rng.standard_normal((2, L)) / L).astype(np.float32)
    err = oracle.normwise_error(oracle.refkernel_f32(g, x, reverse), oracle.scan_f64(g, x, reverse))
    assert err < 1e-5


def test_refkernel_ignores_first_gate():
    """full_scan.cu:96 -- thread 0 of chunk 0 uses 1 in place of the first gate."""
    rng = np.random.default_rng(3)
    g = (0.9 + 0.1 * rng.random((2, 64))).astype(np.float32)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    g2 = g.copy()
    g2[:, 0] = np.nan
    np.testing.assert_array_equal(oracle.refkernel_f32(g2, x), oracle.refkernel_f32(g, x))
    g3 = g.copy()
    g3[:, -1] = np.nan
    np.testing.assert_array_equal(oracle.refkernel_f32(g3, x, True), oracle.refkernel_f32(g, x, True))


def test_refkernel_rejects_what_the_reference_rejects():
    with pytest.raises(ValueError):
        oracle.refkernel_f32(np.ones((1, 48)), np.ones((1, 48)))


def test_normwise_error_definition():
    ref = np.array([[1.0, -4.0, 2.0]])
    assert oracle.normwise_error(ref + np.array([[0.0, 0.4, 0.0]]), ref) == pytest.approx(0.1)
    assert oracle.normwise_error(np.zeros((1, 3)), np.zeros((1, 3))) == 0.0


# ---------------------------------------------------------------- channel-last helpers
def _loop_axis1(g, x, reverse=False):
    """The channel-last definition written out: state per (batch, column), stepped along
    axis 1 (seqlen) in processing order."""
    B, L, D = x.shape
    y = np.empty_like(x)
    state = np.zeros((B, D))
    ts = range(L - 1, -1, -1) if reverse else range(L)
    for t in ts:
        state = g[:, t, :] * state + x[:, t, :]
        y[:, t, :] = state
    return y


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 5, 3), (3, 33, 8), (1, 100, 17)])
def test_channel_last_matches_direct_loop_along_seqlen(shape, reverse):
    rng = np.random.default_rng(sum(shape))
    g = rng.uniform(-1.2, 1.2, size=shape)
    x = rng.standard_normal(size=shape)
    y = oracle.scan_f64_channel_last(g, x, reverse)
    np.testing.assert_allclose(y, _loop_axis1(g, x, reverse), rtol=1e-13, atol=1e-13)


def test_channel_last_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 40, 6))
    ones = np.ones_like(x)
    np.testing.assert_allclose(oracle.scan_f64_channel_last(ones, x), np.cumsum(x, axis=1),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.scan_f64_channel_last(ones, x, reverse=True),
                               np.cumsum(x[:, ::-1], axis=1)[:, ::-1], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(oracle.scan_f64_channel_last(np.zeros_like(x), x), x)


@pytest.mark.parametrize("shape", [(1, 1, 2), (2, 7, 3), (1, 32, 5)])
def test_channel_last_backward_matches_torch_autograd(shape):
    rng = np.random.default_rng(7 + sum(shape))
    g = rng.uniform(-1.2, 1.2, size=shape)
    x = rng.standard_normal(size=shape)
    go = rng.standard_normal(size=shape)
    gt = torch.tensor(g, requires_grad=True)
    xt = torch.tensor(x, requires_grad=True)
    state = torch.zeros(shape[0], shape[2], dtype=torch.float64)
    outs = []
    for t in range(shape[1]):
        state = gt[:, t, :] * state + xt[:, t, :]
        outs.append(state)
    (torch.stack(outs, dim=1) * torch.tensor(go)).sum().backward()
    gg, gx = oracle.scan_bwd_f64_channel_last(g, oracle.scan_f64_channel_last(g, x), go)
    np.testing.assert_allclose(gx, xt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gg, gt.grad.numpy(), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- dimwise (contraction scan)
def _contraction_model(Ax, Bx, kBh, wq1, G, C):
    """The reference's own Python model of the contraction scan (scans/contraction_scan.py:
    98-142), restated in float64 torch: (batch, seqlen, dim) layout, a per-token loop inside
    each group, torch.max over the scores per dim. kBh holds k per (batch, group, dim) and
    wq1 the factor that makes q from v (the model's arguments kBh and Wq; the kernel's
    (1+Wk)*Bh and (1+Wq) are passed in, as the model's caller would)."""
    B, T, Dm = Ax.shape
    per, wc = T // G, G // C
    out = torch.empty(B, T, Dm, dtype=torch.float64)
    carry = None
    for c in range(C):
        ends = []
        for gi in range(wc):
            first = (c * wc + gi) * per
            state = torch.zeros(B, Dm, dtype=torch.float64)
            for t in range(first, first + per):
                prev = carry if (c > 0 and gi == 0 and t == first) else state
                state = Ax[:, t] * prev + Bx[:, t]
                out[:, t] = state
            ends.append(state)
        v = torch.stack(ends, dim=1)
        q = wq1 * v
        r = v.clone()
        for gi in range(1, wc - 1):
            best, idx = torch.max(q[:, gi:gi + 1, :] * kBh[:, :gi, :], dim=1)
            r[:, gi] = torch.gather(v, 1, idx[:, None, :])[:, 0] * best + v[:, gi]
        for gi in range(1, wc):
            s = (c * wc + gi) * per
            out[:, s:s + per] += r[:, gi - 1][:, None, :]
        carry = out[:, (c + 1) * wc * per - 1]
    return out


@pytest.mark.parametrize("L", [64, 128, 256, 512, 1024, 2048, 4096, 8192])
def test_dimwise_matches_the_reference_python_model(L):
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    G = W * C
    rng = np.random.default_rng(L)
    B, D = 2, 3
    a = 0.99 + 0.01 * rng.random((B, D, L))  # scans/contraction_scan.py:154-159 distributions
    x = rng.standard_normal((B, D, L)) / G
    bh = rng.standard_normal((B, D, G)) / G
    wq = 0.01 * rng.random(D)
    wk = 0.01 * rng.random(D)
    got = oracle.dimwise_f64(a, x, bh, wq, wk)
    kbh = torch.tensor(((1 + wk)[None, :, None] * bh[:, :, :W]).transpose(0, 2, 1))
    want = _contraction_model(torch.tensor(a.transpose(0, 2, 1)),
                              torch.tensor(x.transpose(0, 2, 1)), kbh,
                              torch.tensor(1 + wq)[None, None, :], G, C)
    np.testing.assert_allclose(got, want.numpy().transpose(0, 2, 1), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("L", [64, 512, 4096, 16384])
def test_dimwise_closed_form_with_unit_gates_and_zero_keys(L):
    """Gates 1, k = 0: every score is 0 > -1e10, so m = 0 and r[g] = v[g]. Then each group
    is its own cumsum (group 0 from the chunk carry) plus the previous group's total."""
    W, P, C = oracle.DIMWISE_GEOMETRY[L]
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, L))
    ones = np.ones_like(x)
    got = oracle.dimwise_f64(ones, x, np.zeros((2, 3, W * C)), np.zeros(3), np.zeros(3))
    want = np.empty_like(x)
    carry = np.zeros((2, 3))
    for c in range(C):
        cs = np.cumsum(x[:, :, c * W * P:(c + 1) * W * P].reshape(2, 3, W, P), axis=-1)
        cs[:, :, 0] += carry[..., None]
        totals = cs[..., -1].copy()
        cs[:, :, 1:] += totals[:, :, :-1, None]
        want[:, :, c * W * P:(c + 1) * W * P] = cs.reshape(2, 3, W * P)
        carry = cs[:, :, -1, -1]
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_dimwise_two_groups_is_a_cumsum():
    """seqlen 64: two groups and no selection, so with gates 1 the output is cumsum(x)."""
    x = np.random.default_rng(4).standard_normal((1, 2, 64))
    got = oracle.dimwise_f64(np.ones_like(x), x, np.ones((1, 2, 2)), np.zeros(2), np.zeros(2))
    np.testing.assert_allclose(got, np.cumsum(x, axis=-1), rtol=1e-12, atol=1e-12)


def test_dimwise_ties_pick_the_first_group():
    """Equal keys and q > 0: all scores tie, the first strict maximum is group 0, so
    r[g] = (k q[g]) v[0] + v[g] with q[g] = v[g]."""
    L = 1024
    W, P, _ = oracle.DIMWISE_GEOMETRY[L]
    x = 0.5 + np.random.default_rng(5).random((1, 1, L))  # positive: v > 0
    k = 0.25
    got = oracle.dimwise_f64(np.ones_like(x), x, np.full((1, 1, W), k), np.zeros(1), np.zeros(1))
    cs = np.cumsum(x.reshape(W, P), axis=-1)
    v = cs[:, -1]
    r = v.copy()
    r[1:W - 1] = (k * v[1:W - 1]) * v[0] + v[1:W - 1]
    cs[1:] += r[:-1, None]
    np.testing.assert_allclose(got.reshape(W, P), cs, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- fused softplus gates
@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 3, 17), (1, 2, 64)])
def test_softplus_gate_scan_matches_torch_autograd(shape):
    """gates = exp(-softplus(z) * rate[d]) through torch's own softplus and exp, a serial
    loop, and float64 autograd: values and all three gradients."""
    rng = np.random.default_rng(sum(shape))
    z = rng.standard_normal(shape) * 3
    rate = rng.uniform(0.01, 2.0, size=shape[1])
    x = rng.standard_normal(shape)
    go = rng.standard_normal(shape)
    zt = torch.tensor(z, requires_grad=True)
    rt = torch.tensor(rate, requires_grad=True)
    xt = torch.tensor(x, requires_grad=True)
    gates = torch.exp(-torch.nn.functional.softplus(zt) * rt[None, :, None])
    y = _torch_serial_scan(gates, xt)
    (y * torch.tensor(go)).sum().backward()
    want_y = y.detach().numpy()
    np.testing.assert_allclose(oracle.scan_softplus_f64(z, rate, x), want_y, rtol=1e-12,
                               atol=1e-12)
    gz, gr, gx = oracle.scan_bwd_softplus_f64(z, rate, want_y, go)
    np.testing.assert_allclose(gx, xt.grad.numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gz, zt.grad.numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gr, rt.grad.numpy(), rtol=1e-11, atol=1e-11)


def test_softplus_gates_limits():
    z = np.array([[[-50.0, 0.0, 50.0]]])
    g = oracle.softplus_gates_f64(z, np.array([2.0]))
    np.testing.assert_allclose(g, [[[np.exp(-2 * np.log1p(np.exp(-50.0))), 0.25, np.exp(-100.0)]]],
                               rtol=1e-12)
