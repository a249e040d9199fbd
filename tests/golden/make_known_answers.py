"""Writes tests/golden/known_answers.json: known-answer vectors for the scan, computed in
exact rational arithmetic (fractions.Fraction), independent of any floating-point code.

The reference (saeeddhqan/fpscan) ships no golden vectors; its only known-answer case is the
all-ones run of scans/full_scan.py:54-82 (y[t] = t + 1), included here as "all_ones". The
other cases are chosen so that a dropped term, a wrong shift or a transposed operand changes
the answer:

  segmented_cumsum  gates in {0, 1}, small integer tokens: y is a cumulative sum that restarts
                    wherever a gate is 0 (the gate at a restart multiplies the carry by 0).
                    Every partial result is a small integer, so fp32/fp16/bf16 kernels must
                    reproduce it bit for bit in any combine order.
  dyadic            gates and tokens with few significant bits (k/4, k/8): exact answers, stored
                    rounded once to float64; L = 32 and 64 (the kernel's short-row
                    range) forward and reverse.
  backward          grad_tokens / grad_gates for dyadic inputs, from the definitions
                    grad_tokens[t] = grad_out[t] + gates[t+1] grad_tokens[t+1] (gates[L] = 1),
                    grad_gates[t] = grad_tokens[t] y[t-1] (y[-1] = 0), i.e. the gradients of
                    sum(grad_out * y), which fpscan/ops.py:69-83 computes.

Usage: python tests/golden/make_known_answers.py   (deterministic: fixed seeds)
"""
from __future__ import annotations

import json
import os
import random
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "known_answers.json")


def scan_exact(g, x, reverse=False):
    n = len(x)
    y = [Fraction(0)] * n
    acc = Fraction(0)
    order = range(n - 1, -1, -1) if reverse else range(n)
    for t in order:
        acc = g[t] * acc + x[t]
        y[t] = acc
    return y


def backward_exact(g, y, go):
    n = len(g)
    gx = [Fraction(0)] * n
    gg = [Fraction(0)] * n
    acc = Fraction(0)
    for t in range(n - 1, -1, -1):
        nxt = g[t + 1] if t + 1 < n else Fraction(1)
        acc = nxt * acc + go[t]
        gx[t] = acc
        gg[t] = acc * (y[t - 1] if t > 0 else Fraction(0))
    return gg, gx


def enc(vals):
    """Inputs: exact, as short 'p/q' strings."""
    return [str(v) for v in vals]


def res(vals):
    """Expected outputs: the exact value rounded once to the nearest float64 (Fraction ->
    float rounds correctly)."""
    return [float(v) for v in vals]


def case_rows(rng, rows, L, gate_choices, token_choices):
    gs, xs = [], []
    for _ in range(rows):
        gs.append([rng.choice(gate_choices) for _ in range(L)])
        xs.append([rng.choice(token_choices) for _ in range(L)])
    return gs, xs


def main():
    rng = random.Random(20261201)
    cases = []

    # scans/full_scan.py:54-82: all-ones gates and tokens -> y[t] = t + 1
    L = 32
    g = [[Fraction(1)] * L for _ in range(4)]
    x = [[Fraction(1)] * L for _ in range(4)]
    cases.append(dict(name="all_ones", seqlen=L, gates=[enc(r) for r in g],
                      tokens=[enc(r) for r in x],
                      forward=[res(scan_exact(a, b)) for a, b in zip(g, x)],
                      reverse=[res(scan_exact(a, b, True)) for a, b in zip(g, x)]))

    for L in (32, 64, 128, 256, 512, 1024, 2048):
        zero_one = [Fraction(0)] + [Fraction(1)] * 15  # restarts about every 16 steps
        toks = [Fraction(k) for k in range(-3, 4)]
        g, x = case_rows(rng, 3, L, zero_one, toks)
        cases.append(dict(name=f"segmented_cumsum_L{L}", seqlen=L, gates=[enc(r) for r in g],
                          tokens=[enc(r) for r in x],
                          forward=[res(scan_exact(a, b)) for a, b in zip(g, x)],
                          reverse=[res(scan_exact(a, b, True)) for a, b in zip(g, x)]))

    gates_dy = [Fraction(k, 4) for k in (-3, -2, -1, 1, 2, 3, 4)]
    toks_dy = [Fraction(k, 8) for k in range(-8, 9)]
    for L in (32, 64):
        g, x = case_rows(rng, 6, L, gates_dy, toks_dy)
        go = [[rng.choice(toks_dy) for _ in range(L)] for _ in range(6)]
        fwd = [scan_exact(a, b) for a, b in zip(g, x)]
        bwd = [backward_exact(a, y, o) for a, y, o in zip(g, fwd, go)]
        cases.append(dict(name=f"dyadic_L{L}", seqlen=L, gates=[enc(r) for r in g],
                          tokens=[enc(r) for r in x], grad_out=[enc(r) for r in go],
                          forward=[res(r) for r in fwd],
                          reverse=[res(scan_exact(a, b, True)) for a, b in zip(g, x)],
                          grad_gates=[res(b[0]) for b in bwd],
                          grad_tokens=[res(b[1]) for b in bwd]))

    with open(OUT, "w") as f:
        json.dump(dict(generator="tests/golden/make_known_answers.py", cases=cases), f,
                  separators=(",", ":"))
    print(f"wrote {OUT} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
