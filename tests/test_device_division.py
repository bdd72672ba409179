"""The attention epilogues' division by a shared reciprocal (CPU, exact).

fxp_device.h's div_rn_by_recip(a, b, y) with y = RN(1 / b) computes
q = RN(a y), then twice q = RN(q + RN(a - b q) y) with fused multiply-adds,
and claims the bits of the correctly rounded a / b (div_rn) for the ranges
the attention outputs take: a = 0 or |a| in [2^-63, 2^31], b in [1e-6, 2^31].
Each fp32 operation is restated here in exact rational arithmetic (an FMA is
one rounding of the exact a - b q or q + r y) and compared with numpy's
correctly rounded float32 division, on random operands with significands
biased to the ends of [1, 2) (where reciprocal and quotient roundings are
closest to ties) and on the range limits; planted variants (no correction,
a reciprocal off by two ulps) must fail.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np


def _rn32(x: Fraction) -> np.float32:
    """Exact round-to-nearest-even of a rational to binary32 (normal range)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    if Fraction(2) ** (e + 1) <= x:
        e += 1
    m = x / Fraction(2) ** (e - 23)  # in [2^23, 2^24)
    q, r = divmod(m.numerator, m.denominator)
    if 2 * r > m.denominator or (2 * r == m.denominator and q & 1):
        q += 1
    return np.float32(sign * float(Fraction(q) * Fraction(2) ** (e - 23)))


def _f(x) -> Fraction:
    return Fraction(float(x))


def _div_by_recip(a: np.float32, b: np.float32, corrections: int = 2, y_ulps: int = 0) -> np.float32:
    y = np.float32(1.0) / b  # div_rn(1, b)
    for _ in range(y_ulps):  # planted: a reciprocal off by ulps (as v_rcp_f32 may be)
        y = np.nextafter(y, np.float32(np.inf))
    q = _rn32(_f(a) * _f(y))
    for _ in range(corrections):
        r = _rn32(_f(a) - _f(b) * _f(q))
        q = _rn32(_f(r) * _f(y) + _f(q))
    return q


def _operands(n: int, seed: int):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = i % 4
        if kind == 0:
            mb = 1.0 + rng.integers(0, 64) * 2.0 ** -23
        elif kind == 1:
            mb = 2.0 - (1 + rng.integers(0, 64)) * 2.0 ** -23
        else:
            mb = 1.0 + rng.random()
        b = np.float32(mb * 2.0 ** rng.integers(-19, 31))
        kind = i % 3
        if kind == 0:
            ma = 1.0 + rng.integers(0, 64) * 2.0 ** -23
        elif kind == 1:
            ma = 2.0 - (1 + rng.integers(0, 64)) * 2.0 ** -23
        else:
            ma = 1.0 + rng.random()
        a = np.float32((1 if rng.random() < 0.5 else -1) * ma * 2.0 ** rng.integers(-63, 31))
        out.append((a, max(b, np.float32(1e-6))))
    return out


def test_shared_reciprocal_division_is_correctly_rounded():
    pairs = _operands(30000, seed=11)
    lim = [np.float32(2.0 ** -63), np.float32(2.0 ** 31 - 128), np.float32(1.0), np.float32(0.0)]
    den = [np.float32(1e-6), np.float32(2.0 ** 31 - 128), np.float32(1.0), np.float32(3.0)]
    pairs += [(a, b) for a in lim for b in den] + [(-a, b) for a in lim for b in den]
    bad = [(a, b) for a, b in pairs if _div_by_recip(a, b) != np.float32(a) / np.float32(b)]
    assert not bad, bad[:5]


def test_planted_mistakes_are_caught():
    # no correction, and a reciprocal two ulps off with one correction: both
    # must differ from the correctly rounded quotient somewhere in the sample
    pairs = _operands(4000, seed=5)
    for kw in ({"corrections": 0}, {"corrections": 1, "y_ulps": 2}):
        bad = sum(_div_by_recip(a, b, **kw) != np.float32(a) / np.float32(b) for a, b in pairs)
        assert bad > 0, kw
