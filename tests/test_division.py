"""The kernels' division x / d = x * rcp(d) rounds to the same bf16 as torch's IEEE fp32 division
for bf16 operands -- the claim that lets the prologue replace every per-element divide by one
multiply (the reciprocal is computed once per row, by v_rcp_f32, whose result is within 1 ulp of
1/d).

Why it holds: x and d carry 8 significant bits, so x / d is either exact with at most 8 bits (a bf16
value) or at least 2^-17 (relative) away from every bf16 rounding boundary (a boundary needs 9
bits); x * rcp is within 2^-22 of x / d for any rcp within 1 ulp of 1/d. The device formula is
restated here in exact rational arithmetic (every fp32 operation rounded once), with each of the
three fp32 values within 1 ulp of 1/d as the reciprocal, and compared with torch's fp32 division
followed by the bf16 cast, the reference's `logits / scales` and `logits.div_(temperature)`
(core/naive.py:218, :266).
"""

from __future__ import annotations

import random

from fractions import Fraction

import numpy as np
import torch


def rn32(value: Fraction) -> float:
    """Round a rational to the nearest fp32 (ties to even)."""

    approx = np.float32(float(value))
    candidates = {float(approx), float(np.nextafter(approx, np.float32(np.inf))),
                  float(np.nextafter(approx, np.float32(-np.inf)))}
    best = min(candidates, key=lambda c: (abs(Fraction(c) - value),
                                          int(np.float32(c).view(np.uint32)) & 1))

    return best


def reciprocals(d: float):
    """RN(1/d) and its two fp32 neighbours: every value a 1-ulp reciprocal may return."""

    r = np.float32(rn32(Fraction(1) / Fraction(d)))

    return (float(r), float(np.nextafter(r, np.float32(np.inf))), float(np.nextafter(r, np.float32(-np.inf))))


def kernel_divs(x: float, d: float):

    return [rn32(Fraction(x) * Fraction(rcp)) for rcp in reciprocals(d)]


def bf16(v: float) -> float:

    return float(torch.tensor(v, dtype=torch.float32).to(torch.bfloat16))


def reference(x: float, d: float) -> float:

    return float((torch.tensor([x], dtype=torch.bfloat16).float() / torch.tensor([d], dtype=torch.bfloat16).float())
                 .to(torch.bfloat16))


def random_bf16(rng: random.Random, lo_exp: int, hi_exp: int) -> float:

    mantissa = rng.randrange(128, 256)
    value = mantissa * 2.0 ** (rng.randrange(lo_exp, hi_exp) - 7)

    return bf16(value if rng.random() < 0.5 else -value)


def test_random_operands():

    rng = random.Random(0)

    for _ in range(20000):

        x = random_bf16(rng, -20, 20)
        d = abs(random_bf16(rng, -6, 6))
        assert all(bf16(q) == reference(x, d) for q in kernel_divs(x, d)), (x, d)


def test_quotients_near_bf16_midpoints():
    """x = bf16(d * m) with m halfway between two bf16 values, so x / d lies as close to a bf16
    rounding boundary as bf16 operands allow (an exact tie needs 9 significant bits and cannot
    occur)."""

    rng = random.Random(1)

    for _ in range(20000):

        d = abs(random_bf16(rng, -3, 3))
        m = (2 * rng.randrange(128, 256) + 1) * 2.0 ** (rng.randrange(-8, 8) - 8)   # 9-bit odd
        x = bf16(d * m)
        assert all(bf16(q) == reference(x, d) for q in kernel_divs(x, d)), (x, d)


def test_exact_quotients_and_specials():

    for x in (0.0, -0.0, 1.0, -3.0, 96.0, 1.5, float("inf"), float("-inf")):

        for d in (1.0, 2.0, 0.5, 1.25, 3.0):

            for got in (kernel_divs(x, d) if np.isfinite(x) else [x / d]):
                assert bf16(got) == reference(x, d) or (np.isnan(got) and np.isnan(reference(x, d)))
