"""Pin the oracle's scalar numerics (CPU only).

Each oracle function is checked against (1) the reference's own known-answer
values (tests/golden/reference_kats.json), and (2) an independent exact
restatement in Python integers / fractions, by brute force over every fp16
bit pattern and stratified fp32 samples (ties, subnormals, +-0, +-inf, NaN).
A dropped rounding step, a wrong tie rule or a wrong saturation bound fails
one of these.
"""

from __future__ import annotations

import json
import math
import pathlib
from fractions import Fraction

import numpy as np
import pytest

from oracle import numerics as N

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


# --------------------------------------------------------------------------
# independent exact restatements


def exact_float_to_fixed(x: float, b: int, f: int) -> int:
    """RNE_sat_b(x * 2^f) with exact rational arithmetic; NaN -> 0.

    fl32(x * 2^f) only differs from the exact product when it overflows to
    inf, which saturates either way, so exact arithmetic is the definition.
    """
    lo, hi = -(1 << (b - 1)), (1 << (b - 1)) - 1
    if math.isnan(x):
        return 0
    if math.isinf(x):
        return hi if x > 0 else lo
    s = Fraction(x) * (1 << f)
    r = round(s)  # Fraction.__round__ is round-half-even
    return min(max(r, lo), hi)


def exact_int_to_f32(q: int) -> float:
    """Nearest-even fp32 to an integer, via integer arithmetic only."""
    if q == 0:
        return 0.0
    sign = -1 if q < 0 else 1
    a = abs(q)
    nb = a.bit_length()
    if nb <= 24:
        return float(q)
    shift = nb - 24
    m, rem = a >> shift, a & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    if rem > half or (rem == half and (m & 1)):
        m += 1
    return sign * float(m) * 2.0 ** shift


def all_f16() -> np.ndarray:
    return np.arange(1 << 16, dtype=np.uint16).view(np.float16)


def stratified_f32(seed: int = 0, n: int = 4000) -> np.ndarray:
    rng = np.random.default_rng(seed)
    vals = [0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 0.5, -0.5, 1.5, 2.5, -2.5,
            np.float32(1e-45), np.float32(-1e-45), np.float32(3.4028235e38), -np.float32(3.4028235e38)]
    # exact ties at several scales for f = 8/16/32: (k + 1/2) * 2^-f
    for f in (8, 16, 32):
        for k in (-3, -2, -1, 0, 1, 2, 3, 1000, -1001):
            vals.append((k + 0.5) * 2.0 ** -f)
    # values around the int16/int32/int64 saturation edges at f = 16
    for e in (15, 31, 47, 63):
        for d in (-1.0, -0.5, 0.0, 0.5, 1.0):
            vals.append((2.0 ** e + d) / 65536.0)
            vals.append(-(2.0 ** e + d) / 65536.0)
    vals = np.array(vals, dtype=np.float32)
    rnd = (rng.standard_normal(n) * np.exp2(rng.integers(-40, 60, n))).astype(np.float32)
    bits = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate([vals, rnd, bits])


# --------------------------------------------------------------------------
# reference known-answer values


def test_kat_cast_known_values():
    k = KATS["cast_known_values"]
    q = N.float_to_fixed(np.array(k["x_f32"], np.float32), k["int_bits"], k["frac_bits"])
    assert q.dtype == np.int32
    assert q.tolist() == k["q_i32"]


def test_kat_cast_saturation():
    k = KATS["cast_saturation"]
    q = N.float_to_fixed(np.array(k["x_f32"], np.float32), k["int_bits"], k["frac_bits"])
    for v, (lo, hi) in zip(q.tolist(), k["q_bounds"]):
        assert lo <= v <= hi


def test_kat_roundtrips():
    k = KATS["float_roundtrip_lossless"]
    x = np.array(k["x_f32"], np.float32)
    back = N.fixed_to_float(N.float_to_fixed(x, 32, 16), 32, 16)
    assert np.array_equal(back.view(np.uint32), x.view(np.uint32))

    k = KATS["float_roundtrip_rounding"]
    x = np.array(k["x_f32"], np.float32)
    back = N.fixed_to_float(N.float_to_fixed(x, 32, 16), 32, 16).astype(np.float64)
    step = 2.0 ** -16
    assert np.allclose(np.round(back / step) * step - back, 0.0, atol=1e-7)
    assert np.all(np.abs(x.astype(np.float64) - back) <= step / 2 + 1e-7)
    assert np.any(x.astype(np.float64) != back)

    k = KATS["fixed_roundtrip_lossless"]
    q = np.array(k["q_i32"], np.int32)
    assert N.float_to_fixed(N.fixed_to_float(q, 32, 16), 32, 16).tolist() == q.tolist()

    k = KATS["float_roundtrip_frac_bits"]
    x = np.array(k["x_f32"], np.float32)
    for f in k["frac_bits"]:
        back = N.fixed_to_float(N.float_to_fixed(x, 64, f), 32, f)
        assert np.array_equal(back, x)


def test_kat_sums():
    k = KATS["sum_on_q_grid"]
    q = np.array(k["q_i32"], np.int32)
    x = N.fixed_to_float(q.astype(np.int64), 32, 16)
    assert N.float_to_fixed(x, 32, 16).tolist() == q.tolist()
    s = N.fixed_row_sum(N.float_to_fixed(x, 32, 16), 32)
    assert int(s) == k["sum_q"]
    # the fp32 sum of on-grid values equals the fixed-point sum bit for bit
    assert np.float32(x.sum(dtype=np.float32)).view(np.uint32) == N.fixed_to_float(
        np.int64(s), 32, 16).view(np.uint32)

    for name in ("sum_saturates_max", "sum_saturates_min"):
        k = KATS[name]
        q = N.float_to_fixed(np.array(k["x_f32"], np.float32), k["int_bits"], k["frac_bits"])
        assert int(N.fixed_row_sum(q, 32)) == k["sum_q"]

    k = KATS["sum_associativity"]
    a = N.fixed_row_sum(N.float_to_fixed(np.array(k["order_a"], np.float32), 64, 16), 64)
    b = N.fixed_row_sum(N.float_to_fixed(np.array(k["order_b"], np.float32), 64, 16), 64)
    assert int(a) == int(b)
    assert N.fixed_to_float(np.int64(a), 32, 16) == np.float32(k["sum_f32"])
    # and fp16 really is order dependent on these values
    fa = np.float16(0)
    for v in k["order_a"]:
        fa = np.float16(fa + np.float16(v))
    fb = np.float16(0)
    for v in k["order_b"]:
        fb = np.float16(fb + np.float16(v))
    assert fa != fb


# --------------------------------------------------------------------------
# brute force against the exact restatement


@pytest.mark.parametrize("b", [16, 32, 64])
@pytest.mark.parametrize("f", [0, 8, 16, 32])
def test_float_to_fixed_all_f16(b, f):
    x = all_f16()
    q = N.float_to_fixed(x, b, f)
    want = [exact_float_to_fixed(float(v), b, f) for v in x.astype(np.float64)]
    assert q.dtype == N.INT_DTYPE_BY_BITS[b]
    assert q.astype(np.int64).tolist() == want


@pytest.mark.parametrize("b", [16, 32, 64])
@pytest.mark.parametrize("f", [8, 16, 32, 63])
def test_float_to_fixed_stratified_f32(b, f):
    x = stratified_f32(seed=b * 100 + f)
    q = N.float_to_fixed(x, b, f)
    # fl32(x * 2^f) overflowing to inf saturates; exact arithmetic agrees
    want = [exact_float_to_fixed(float(v), b, f) for v in x.astype(np.float64)]
    assert q.astype(np.int64).tolist() == want


def test_float_to_fixed_f64_rounds_to_f32_first():
    # 1 + 2^-30 is not an fp32; rounded to fp32 first it is 1.0 -> 2^16 exactly
    x = np.array([1.0 + 2.0 ** -30, 0.5 + 2.0 ** -17 + 2.0 ** -40], np.float64)
    q = N.float_to_fixed(x, 32, 16)
    assert q.tolist() == [exact_float_to_fixed(float(np.float32(v)), 32, 16) for v in x]
    assert q[0] == 65536


def test_fixed_to_float_exact():
    rng = np.random.default_rng(1)
    qs = [0, 1, -1, 2 ** 24 + 1, 2 ** 24 + 3, 2 ** 60 + 2 ** 36 + 1, -(2 ** 60 + 2 ** 36 + 1),
          2 ** 63 - 1, -(2 ** 63), 2 ** 31 - 1, -(2 ** 31)]
    qs += [int(v) for v in rng.integers(-(2 ** 63), 2 ** 63 - 1, 3000, dtype=np.int64)]
    q = np.array(qs, np.int64)
    for f in (0, 8, 16, 32):
        got = N.fixed_to_float(q, 32, f)
        want = np.array([exact_int_to_f32(v) * 2.0 ** -f for v in qs], np.float64)
        assert np.array_equal(got.astype(np.float64), want)
    # int16 -> f16 output: fp32 value rounded to fp16 (RNE)
    q16 = np.arange(-32768, 32768, dtype=np.int16)
    got = N.fixed_to_float(q16, 16, 8)
    assert np.array_equal(got, (q16.astype(np.float64) / 256.0).astype(np.float32).astype(np.float16))


def test_fixed_row_sum_exact_then_saturate():
    rng = np.random.default_rng(2)
    q = rng.integers(-(2 ** 62), 2 ** 62, (5, 9), dtype=np.int64)
    got = N.fixed_row_sum(q, 64)
    for r in range(5):
        s = sum(int(v) for v in q[r])
        assert int(got[r]) == min(max(s, -(2 ** 63)), 2 ** 63 - 1)
    # exact first, saturate once: +max, +max, -max sums to +max, not a clamp
    # after the second term
    q = np.array([[2 ** 31 - 1, 2 ** 31 - 1, -(2 ** 31 - 1)]], np.int32)
    assert int(N.fixed_row_sum(q, 32)[0]) == 2 ** 31 - 1
    q = np.array([[2 ** 30, 2 ** 30, -(2 ** 30)]], np.int32)
    assert int(N.fixed_row_sum(q, 32)[0]) == 2 ** 30


def test_bf16_rounding_matches_torch():
    import torch

    x = stratified_f32(seed=7)
    got = N.f32_to_bf16(x)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(got[nan] == 0x7FC0)
    back = N.bf16_to_f32(got[~nan])
    assert np.array_equal(back, torch.from_numpy(x[~nan].copy()).to(torch.bfloat16).float().numpy())


def test_exp_scaled_accuracy_and_floor():
    d = np.concatenate([-np.linspace(0, 80, 200001, dtype=np.float64).astype(np.float32),
                        np.float32([-0.0, -1e-30, -0.5, -0.25])])
    # the reduction t = fl(d*fl32(log2e)) costs half an ulp of t plus the
    # constant's own error times |d|, each scaled by ln2 in the result; the
    # polynomial adds a few 1e-8
    t = np.abs(d.astype(np.float64)) * math.log2(math.e)
    const_err = abs(float(N.LOG2E) - math.log2(math.e))
    bound = 2e-7 + math.log(2) * (
        0.5 * np.spacing(t.astype(np.float32)).astype(np.float64)
        + np.abs(d.astype(np.float64)) * const_err) * 1.01
    for f in (0, 16, 32):
        got = N.exp_scaled(d, f).astype(np.float64)
        want = np.exp(d.astype(np.float64)) * 2.0 ** f
        rel = np.abs(got - want) / want
        assert np.all(rel <= bound), (f, float(rel.max()))
    assert N.exp_scaled(np.float32([-80.0001, -np.inf, np.nan, -1000.0]), 16).tolist() == [0, 0, 0, 0]
    assert N.exp_scaled(np.float32([0.0]), 16)[0] == 65536.0
    assert N.exp_scaled(np.float32([0.0]), 0)[0] == 1.0


def test_log_own_accuracy():
    rng = np.random.default_rng(3)
    y = np.concatenate([np.float32([1.0, 2.0, 0.5, 1.41421356, 1.41421357, 2.0 ** -32, 2.0 ** 31]),
                        (np.exp2(rng.uniform(-32, 40, 20000))).astype(np.float32)])
    got = N.log_own(y).astype(np.float64)
    want = np.log(y.astype(np.float64))
    err = np.abs(got - want)
    assert np.all(err <= 4e-7 * np.maximum(1.0, np.abs(want))), err.max()
    assert N.log_own(np.float32([1.0]))[0] == 0.0


def _fma_exact(a, b, c):
    """Correctly rounded fp32 of a*b + c by exact rational arithmetic."""
    from fractions import Fraction
    x = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if x == 0:
        return np.float32(0.0)
    r = np.float32(float(x))  # float(x) rounds the exact value to float64 ...
    # ... so pick among the fp32 neighbours of that guess by exact distance
    cands = [np.nextafter(r, np.float32(-np.inf)), r, np.nextafter(r, np.float32(np.inf))]
    best = None
    for cnd in cands:
        dist = abs(Fraction(float(cnd)) - x)
        key = (dist, int(np.float32(cnd).view(np.uint32)) & 1)  # ties to the even significand
        if best is None or key < best[0]:
            best = (key, cnd)
    return np.float32(best[1])


def test_fma_f32_matches_exact_rounding():
    rng = np.random.default_rng(0)
    # random operands over a wide exponent range
    a = (rng.standard_normal(3000) * 2.0 ** rng.integers(-20, 20, 3000)).astype(np.float32)
    b = (rng.standard_normal(3000) * 2.0 ** rng.integers(-20, 20, 3000)).astype(np.float32)
    c = (rng.standard_normal(3000) * 2.0 ** rng.integers(-40, 40, 3000)).astype(np.float32)
    # integer operands: a*b + c lands exactly on fp32 ties often
    ai = rng.integers(1, 1 << 13, 2000).astype(np.float32)
    bi = rng.integers(1, 1 << 13, 2000).astype(np.float32)
    ci = rng.integers(-(1 << 12), 1 << 12, 2000).astype(np.float32)
    # double-rounding traps: a*b an exact fp32 tie (odd multiple of half an
    # ulp at 2^25), c a tiny nudge of either sign that float64 alone loses
    at = (2.0 * rng.integers(1 << 11, 1 << 12, 1000) + 1).astype(np.float32)   # odd, 12 bits
    bt = (2.0 ** 13 * (2 * rng.integers(1 << 11, 1 << 12, 1000) + 1)).astype(np.float32)
    ct = (rng.choice([-1.0, 1.0], 1000) * 2.0 ** rng.integers(-40, -20, 1000)).astype(np.float32)
    A_ = np.concatenate([a, ai, at]); B_ = np.concatenate([b, bi, bt]); C_ = np.concatenate([c, ci, ct])
    got = N.fma_f32(A_, B_, C_)
    want = np.array([_fma_exact(x, y, z) for x, y, z in zip(A_, B_, C_)], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the trap cases really are ties that plain float64 evaluation gets wrong
    naive = (at.astype(np.float64) * bt + ct).astype(np.float32)
    assert (naive != N.fma_f32(at, bt, ct)).sum() > 100
