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


@pytest.mark.parametrize("c,H", [(0.5, 64), (2.0, 4096), (0.25, 1024), (3.0, 16)])
def test_rms_norm_constant_row_closed_form(c, H):
    x = np.full((3, H), c, np.float32)
    w = np.linspace(-2, 2, H).astype(np.float32)
    y, _ = R.rms_norm(x, w, 1e-6, "f32", 32, 16)
    # c^2 is on the Q16.16 grid and H*q is exact in fp32, so mean_sq == c^2
    rrms = _f32_rrms(c * c, 1e-6)
    want = (F32(c) * w) * rrms
    assert np.array_equal(y, np.broadcast_to(want, y.shape))


def test_rms_norm_sum_is_integer_fixed_point():
    # one element whose square is off-grid: the sum uses RNE(v^2 * 2^16)
    x = np.array([[1.0 + 2.0 ** -10, 0.0, 0.0, 0.0]], np.float32)
    w = np.ones(4, np.float32)
    y, _ = R.rms_norm(x, w, 0.0, "f32", 32, 16)
    q = round((1.0 + 2.0 ** -10) ** 2 * 65536)  # exact square, then RNE
    ms = F32(F32(q) * F32(2.0 ** -16)) / F32(4.0)
    assert y[0, 0] == F32(x[0, 0] * _f32_rrms(float(ms), 0.0))


def _rand(shape, seed, lo=-0.5, hi=0.5, scale=1.0):
    rng = np.random.default_rng(seed)
    return ((rng.random(shape) * (hi - lo) + lo) * scale).astype(np.float32)


@pytest.mark.parametrize("shape", [(2, 7), (3, 16), (4, 31)])
def test_rms_norm_tolerance_vs_reference_fp32(shape):
    # fxpr_vllm/_tests/test_rms_norm.py:39-57 (inputs within Q16.16 range)
    x = _rand(shape, 0, scale=32.0)
    w = _rand(shape[1:], 1, scale=4.0)
    y, _ = R.rms_norm(x, w, 1e-6, "f32", 32, 16)
    ref = R.rms_norm_reference_fp32(x, w, 1e-6)
    assert np.allclose(y, ref, atol=5e-4, rtol=5e-4)


@pytest.mark.parametrize("io,tol", [("f32", 5e-4), ("f16", 5e-3), ("bf16", 2e-2)])
@pytest.mark.parametrize("shape", [(2, 16), (4, 64)])
def test_rms_norm_native_dtype_tolerance(io, tol, shape):
    # fxpr_vllm/_tests/test_rms_norm.py:60-97
    x32 = _rand(shape, 2, scale=4.0)
    w32 = _rand(shape[1:], 3, scale=2.0)
    x, w = N.store(x32, io), N.store(w32, io)
    y, _ = R.rms_norm(x, w, 1e-6, io, 32, 16)
    ref = N.round_io(R.rms_norm_reference_fp32(N.load(x, io), N.load(w, io), 1e-6).astype(np.float32), io)
    assert np.allclose(N.load(y, io), ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("io,tol", [("f32", 5e-4), ("f16", 5e-3), ("bf16", 2e-2)])
def test_rms_norm_residual_writeback(io, tol):
    # fxpr_vllm/_tests/test_rms_norm.py:100-130
    x32, r32, w32 = _rand((4, 32), 11, scale=2.0), _rand((4, 32), 12, scale=2.0), _rand((32,), 13, scale=2.0)
    x, r, w = N.store(x32, io), N.store(r32, io), N.store(w32, io)
    y, new_r = R.rms_norm(x, w, 1e-6, io, 32, 16, residual=r)
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
    y, _ = R.rms_norm(x, np.ones(5, np.float32), k["eps"], "f32", 32, 16)
    assert np.array_equal(y[1], y[0][perm])


@pytest.mark.parametrize("b,f", [(32, 16), (64, 32), (64, 16), (16, 8)])
def test_rms_norm_row_order_free(b, f):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 257)).astype(np.float32)
    w = rng.standard_normal(257).astype(np.float32)
    p = rng.permutation(257)
    y, _ = R.rms_norm(x, w, 1e-6, "f32", b, f)
    yp, _ = R.rms_norm(x[:, p], w[p], 1e-6, "f32", b, f)
    assert np.array_equal(yp, y[:, p])


def test_rms_norm_int32_saturation_is_defined():
    # |v| > 181 saturates each q at Q16.16 / int32; the sum then saturates too
    x = np.full((1, 8), 200.0, np.float32)
    y, _ = R.rms_norm(x, np.ones(8, np.float32), 0.0, "f32", 32, 16)
    ms = F32(F32(2 ** 31 - 1) * F32(2.0 ** -16)) / F32(8.0)
    assert y[0, 0] == F32(F32(200.0) * _f32_rrms(float(ms), 0.0))


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


def test_log_softmax_int32_sum_saturates():
    # 40000 equal logits: S = 40000 * 2^16 > INT32_MAX, saturates
    x = np.zeros((1, 40000), np.float32)
    y = R.log_softmax(x, "f32", "f32", 32, 16)
    want = -F32(N.log_own(np.float32([F32(2 ** 31 - 1) * F32(2.0 ** -16)]))[0])
    assert y[0, 0] == want
    y64 = R.log_softmax(x, "f32", "f32", 64, 16)
    assert abs(float(y64[0, 0]) + math.log(40000)) < 1e-5


def test_log_softmax_bf16_io_and_special_rows():
    x = np.array([[-np.inf] * 4, [np.nan, 0, 1, 2], [0, -np.inf, 1, -np.inf]], np.float32)
    y = R.log_softmax(N.store(x, "bf16"), "bf16", "f32", 32, 16)
    assert np.all(np.isnan(y[0])) and np.all(np.isnan(y[1]))
    assert y[2, 1] == -np.inf and y[2, 3] == -np.inf
    ref = np.array([0, 1]) - math.log(1 + math.e)
    assert np.allclose(y[2, [0, 2]], ref, atol=1e-4)
