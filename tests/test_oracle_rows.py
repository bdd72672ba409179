"""Pin the oracle's RMSNorm and log-softmax (CPU only).

RMSNorm: closed form on constant rows (every step exact, so the result is the
IEEE evaluation of w*c/sqrt(c^2+eps)), the reference's own fp32 tolerance tests
(fxpr_vllm/_tests/test_rms_norm.py:39-130), exact permutation equivariance
(:133-151) and residual write-back.
Log-softmax (build-defined): one-hot row gives y_max = 0 exactly, constant row
gives -ln N to quantisation accuracy, brute force against float64 on random
rows, permutation equivariance, saturation behaviour.
"""

from __future__ import annotations

import json
import math
import pathlib

import numpy as np
import pytest

from oracle import numerics as N
from oracle import rows as R

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())
F32 = np.float32


def _f32_rrms(ms: float, eps: float) -> np.float32:
    t = F32(F32(ms) + F32(eps))
    return F32(F32(1.0) / F32(np.sqrt(t)))


@pytest.mark.parametrize("c,H", [(0.5, 64), (2.0, 4096), (0.25, 1024), (3.0, 16), (1500.0, 4096),
                                 (-7.0e5, 256), (3.0e-9, 128)])
def test_rms_norm_constant_row_closed_form(c, H):
    # s = c * 2^-e is exact, fl32(s^2) * 2^40 is an integer, H * that is
    # exact, so mean_sq == fl32(c^2) for every magnitude (H a power of two)
    x = np.full((3, H), c, np.float32)
    w = np.linspace(-2, 2, H).astype(np.float32)
    y, _ = R.rms_norm(x, w, 1e-6, "f32")
    rrms = _f32_rrms(F32(c) * F32(c), 1e-6)
    want = (F32(c) * w) * rrms
    assert np.array_equal(y, np.broadcast_to(want, y.shape))


def test_rms_norm_off_grid_square_is_not_quantised_away():
    # (1 + 2^-10)^2 needs 21 significant bits: the sum keeps all of them, and
    # its mean over H = 4 is exact
    x = np.array([[1.0 + 2.0 ** -10, 0.0, 0.0, 0.0]], np.float32)
    y, _ = R.rms_norm(x, np.ones(4, np.float32), 0.0, "f32")
    ms = F32((1.0 + 2.0 ** -10) ** 2 / 4)
    assert float(ms) == (1.0 + 2.0 ** -10) ** 2 / 4
    assert y[0, 0] == F32(x[0, 0] * _f32_rrms(float(ms), 0.0))
    assert y[0, 1] == 0.0


def _rand(shape, seed, lo=-0.5, hi=0.5, scale=1.0):
    rng = np.random.default_rng(seed)
    return ((rng.random(shape) * (hi - lo) + lo) * scale).astype(np.float32)


@pytest.mark.parametrize("shape", [(2, 7), (3, 16), (4, 31)])
def test_rms_norm_tolerance_vs_reference_fp32(shape):
    # fxpr_vllm/_tests/test_rms_norm.py:39-57
    x = _rand(shape, 0, scale=32.0)
    w = _rand(shape[1:], 1, scale=4.0)
    y, _ = R.rms_norm(x, w, 1e-6, "f32")
    ref = R.rms_norm_reference_fp32(x, w, 1e-6)
    assert np.allclose(y, ref, atol=5e-4, rtol=5e-4)


def realistic_rows(H=4096, seed=0):
    """Rows at residual-stream magnitudes: RMS 3, 5, 20, 100 and 1e4, a tiny
    row (RMS 1e-3), and an N(0, 0.5) row with one channel at 1500."""
    rng = np.random.default_rng(seed)
    rows = [rng.standard_normal(H) * s for s in (3.0, 5.0, 20.0, 100.0, 1.0e4, 1.0e-3)]
    spike = rng.standard_normal(H) * 0.5
    spike[H // 3] = 1500.0
    rows.append(spike)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("io,tol", [("f32", 4e-6), ("f16", 5e-3), ("bf16", 2e-2)])
@pytest.mark.parametrize("residual", [False, True])
def test_rms_norm_realistic_magnitudes_vs_float64(io, tol, residual):
    # The reference sums v*v in fp32 and never saturates
    # (fxpr_vllm/_triton/rms_norm.py:4, 49-53); at these magnitudes the
    # integer sum must stay within the reference's own tolerances
    # (_tests/test_rms_norm.py: 5e-4 fp32, 5e-3 f16, 2e-2 bf16) and, for fp32
    # I/O, within a few fp32 ulps of a float64 RMSNorm.
    x32 = realistic_rows()
    r32 = realistic_rows(seed=1) * np.float32(0.5) if residual else None
    w32 = (np.random.default_rng(2).standard_normal(x32.shape[1]) * 0.1 + 1).astype(np.float32)
    x, w = N.store(x32, io), N.store(w32, io)
    r = None if r32 is None else N.store(r32, io)
    y, new_r = R.rms_norm(x, w, 1e-6, io, residual=r)
    u = N.load(new_r if r is not None else x, io).astype(np.float64)
    v = N.load(x, io).astype(np.float64) + (0 if r is None else N.load(r, io).astype(np.float64))
    ref = u * N.load(w, io) / np.sqrt((v * v).mean(axis=-1, keepdims=True) + 1e-6)
    got = N.load(y, io).astype(np.float64)
    assert np.all(np.abs(got - ref) <= tol * np.abs(ref) + tol * 1e-3 * np.abs(ref).max(axis=-1, keepdims=True))


def test_rms_norm_planted_mistakes_fail_the_magnitude_check(monkeypatch):
    # the checks above catch a wrong per-row exponent, a sum fraction too
    # coarse to keep the small channels next to a spike, and a mean scaled by
    # e instead of 2e
    x = realistic_rows()
    w = np.ones(x.shape[1], np.float32)
    ref = (x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6))

    def worst():
        y, _ = R.rms_norm(x, w, 1e-6, "f32")
        return float(np.max(np.abs(y - ref) / np.abs(ref).max(-1, keepdims=True)))

    assert worst() < 4e-6
    real_exp = R.rms_row_exponent
    monkeypatch.setattr(R, "rms_row_exponent", lambda v: (np.zeros_like(real_exp(v)[0]), real_exp(v)[1]))
    assert worst() > 1e-3
    monkeypatch.setattr(R, "rms_row_exponent", real_exp)
    monkeypatch.setattr(R, "RMS_SUM_FRAC", 12)
    assert worst() > 4e-6
    monkeypatch.setattr(R, "RMS_SUM_FRAC", 40)
    orig_ldexp = np.ldexp
    monkeypatch.setattr(R.np, "ldexp", lambda a, k: orig_ldexp(a, k // 2 if np.ndim(k) == 1 else k))
    assert worst() > 1e-3


def test_rms_norm_scale_invariance_is_exact():
    # with eps = 0, scaling a row by 2^k scales mean_sq by 2^(2k) exactly
    # (the per-row exponent absorbs it), so y is bit-identical
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4, 777)) * np.array([[1e-3], [1.0], [50.0], [1e5]])).astype(np.float32)
    w = rng.standard_normal(777).astype(np.float32)
    y0, _ = R.rms_norm(x, w, 0.0, "f32")
    for k in (-40, -7, 1, 9, 30):
        yk, _ = R.rms_norm(np.ldexp(x, k).astype(np.float32), w, 0.0, "f32")
        assert np.array_equal(yk, y0), k


def test_rms_norm_special_rows():
    H = 8
    x = np.zeros((6, H), np.float32)
    x[1] = 2.0 ** -140                     # subnormal row
    x[2] = 2.0 ** -70                      # mean square 2^-140, a subnormal fp32
    x[3] = 1.0e30                          # mean square overflows fp32 (as the reference's sum)
    x[4, 0], x[4, 1:] = np.inf, 1.0
    x[5, 0], x[5, 1:] = np.nan, 1.0
    w = np.full(H, 2.0, np.float32)
    y, _ = R.rms_norm(x, w, 1e-6, "f32")
    assert np.array_equal(y[0], np.zeros(H, np.float32))
    assert np.array_equal(y[1], (x[1] * w) * _f32_rrms(0.0, 1e-6))
    y0, _ = R.rms_norm(x[2:3], w, 0.0, "f32")
    assert np.array_equal(y0[0], w * F32(1.0))
    assert np.array_equal(y[3], np.zeros(H, np.float32))
    assert np.isnan(y[4, 0]) and np.array_equal(y[4, 1:], np.zeros(H - 1, np.float32))
    assert np.all(np.isnan(y[5]))


@pytest.mark.parametrize("io,tol", [("f32", 5e-4), ("f16", 5e-3), ("bf16", 2e-2)])
@pytest.mark.parametrize("shape", [(2, 16), (4, 64)])
def test_rms_norm_native_dtype_tolerance(io, tol, shape):
    # fxpr_vllm/_tests/test_rms_norm.py:60-97
    x32 = _rand(shape, 2, scale=4.0)
    w32 = _rand(shape[1:], 3, scale=2.0)
    x, w = N.store(x32, io), N.store(w32, io)
    y, _ = R.rms_norm(x, w, 1e-6, io)
    ref = N.round_io(R.rms_norm_reference_fp32(N.load(x, io), N.load(w, io), 1e-6).astype(np.float32), io)
    assert np.allclose(N.load(y, io), ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("io,tol", [("f32", 5e-4), ("f16", 5e-3), ("bf16", 2e-2)])
def test_rms_norm_residual_writeback(io, tol):
    # fxpr_vllm/_tests/test_rms_norm.py:100-130
    x32, r32, w32 = _rand((4, 32), 11, scale=2.0), _rand((4, 32), 12, scale=2.0), _rand((32,), 13, scale=2.0)
    x, r, w = N.store(x32, io), N.store(r32, io), N.store(w32, io)
    y, new_r = R.rms_norm(x, w, 1e-6, io, residual=r)
    expected_r = N.store(N.load(x, io) + N.load(r, io), io)
    assert np.array_equal(np.asarray(new_r).view(np.uint8), np.asarray(expected_r).view(np.uint8))
    # output normalises the stored (rounded) residual
    ref = R.rms_norm_reference_fp32(N.load(new_r, io), N.load(w, io), 1e-6).astype(np.float32)
    assert np.allclose(N.load(y, io), N.round_io(ref, io), atol=tol, rtol=tol)


def test_rms_norm_permutation_equivariance_kat():
    k = KATS["rms_norm_associativity"]
    xa = np.array(k["x_f32"], np.float32)
    perm = np.array(k["perm"])
    x = np.stack([xa, xa[perm]])
    y, _ = R.rms_norm(x, np.ones(5, np.float32), k["eps"], "f32")
    assert np.array_equal(y[1], y[0][perm])


def test_rms_norm_row_order_free():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 257)) * np.array([[1.0], [300.0], [1e-4]])).astype(np.float32)
    w = rng.standard_normal(257).astype(np.float32)
    p = rng.permutation(257)
    y, _ = R.rms_norm(x, w, 1e-6, "f32")
    yp, _ = R.rms_norm(x[:, p], w[p], 1e-6, "f32")
    assert np.array_equal(yp, y[:, p])


# --------------------------------------------------------------------------
# log-softmax


@pytest.mark.parametrize("b,f", [(32, 16), (64, 32), (32, 8)])
def test_log_softmax_one_hot_exact(b, f):
    x = np.zeros((2, 1000), np.float32)
    x[0, 17] = 30.0
    x[1, 999] = 40.0
    y = R.log_softmax(x, "f32", "f32", b, f)
    # e^-30 * 2^f < 1/2 for f <= 32: the sum is exactly 2^f, ln 1 = 0
    assert y[0, 17] == 0.0 and y[1, 999] == 0.0
    assert y[0, 0] == -30.0 and y[1, 0] == -40.0


@pytest.mark.parametrize("V", [1, 7, 1000, 32768])
def test_log_softmax_constant_row(V):
    x = np.full((1, V), 3.25, np.float32)
    y = R.log_softmax(x, "f32", "f32", 64, 32)
    assert np.all(y == y[0, 0])
    assert abs(float(y[0, 0]) + math.log(V)) < 2e-6 * max(1.0, math.log(V))


@pytest.mark.parametrize("b,f", [(32, 16), (64, 32)])
def test_log_softmax_vs_float64(b, f):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((8, 513)) * 4).astype(np.float32)
    y = R.log_softmax(x, "f32", "f32", b, f).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd - (xd.max(1, keepdims=True) + np.log(np.exp(xd - xd.max(1, keepdims=True)).sum(1, keepdims=True)))
    # quantising each weight at 2^-f costs <= V*2^-(f+1) in the sum (>= 1)
    tol = 513 * 2.0 ** -(f + 1) + 4e-6
    assert np.max(np.abs(y - ref)) < tol


def test_log_softmax_permutation_equivariance():
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((4, 300)) * 4).astype(np.float32)
    p = rng.permutation(300)
    y = R.log_softmax(x, "f32", "f32", 32, 16)
    assert np.array_equal(R.log_softmax(x[:, p], "f32", "f32", 32, 16), y[:, p])


@pytest.mark.parametrize("b,f", [(32, 16), (16, 8), (64, 32), (64, 63), (32, 0)])
@pytest.mark.parametrize("V", [40000, 128256])
def test_log_softmax_flat_row_never_saturates(b, f, V):
    # every term is 2^f (qmax for (64, 63)); the exact sum V * term exceeds
    # the term's width but is never clamped, so y = -ln V up to log_own's
    # accuracy; (64, 63) sums beyond 64 bits
    x = np.zeros((1, V), np.float32)
    y = R.log_softmax(x, "f32", "f32", b, f)
    assert np.all(y == y[0, 0])
    assert abs(float(y[0, 0]) + math.log(V)) < 4e-6 * math.log(V)
    term = min(2 ** f, 2 ** (b - 1) - 1)
    want = -(F32(0.0) + N.log_own(np.float32([N.int_to_f32(V * term) * F32(2.0 ** -f)]))[0])
    assert y[0, 0] == want


def test_int_to_f32_rounding():
    # ties to even, carries into the next binade, 128-bit values
    assert N.int_to_f32(2 ** 24 + 1) == F32(2 ** 24)
    assert N.int_to_f32(2 ** 24 + 3) == F32(2 ** 24 + 4)
    assert N.int_to_f32(2 ** 90 + 2 ** 66) == F32(2 ** 90)
    assert N.int_to_f32(2 ** 90 + 2 ** 66 + 1) == F32(2 ** 90 + 2 ** 67)
    assert N.int_to_f32(2 ** 95 - 1) == F32(2 ** 95)
    rng = np.random.default_rng(0)
    for n in rng.integers(1, 2 ** 62, 1000):
        assert N.int_to_f32(int(n)) == np.float32(np.int64(n))


def test_log_softmax_bf16_io_and_special_rows():
    x = np.array([[-np.inf] * 4, [np.nan, 0, 1, 2], [0, -np.inf, 1, -np.inf]], np.float32)
    y = R.log_softmax(N.store(x, "bf16"), "bf16", "f32", 32, 16)
    assert np.all(np.isnan(y[0])) and np.all(np.isnan(y[1]))
    assert y[2, 1] == -np.inf and y[2, 3] == -np.inf
    ref = np.array([0, 1]) - math.log(1 + math.e)
    assert np.allclose(y[2, [0, 2]], ref, atol=1e-4)
