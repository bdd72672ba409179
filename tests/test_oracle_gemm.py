"""Pin the oracle's fixed-point GEMM (CPU only).

Exact against Python-integer matmul on small-integer inputs (tile dots exact
in fp32, so the per-tile quantisation and the integer accumulation are fully
determined), wrap-around and saturation of the accumulator, K-tile
permutation invariance (fxpr_vllm/_tests/test_gemm.py:214-242), tolerance
against float64 matmul on random data (test_gemm.py tolerances :91-95), and a
planted-mistake check that a dropped quantisation step is caught.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gemm as G
from oracle import numerics as N


def int_inputs(M, K, Nn, seed, lo=-2, hi=2):
    rng = np.random.default_rng(seed)
    return (rng.integers(lo, hi + 1, (M, K)).astype(np.float32),
            rng.integers(lo, hi + 1, (K, Nn)).astype(np.float32))


@pytest.mark.parametrize("io", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("b,f", [(32, 16), (64, 16), (16, 8), (64, 32)])
def test_exact_on_small_integers(io, b, f):
    a, bb = int_inputs(9, 300, 11, seed=1)
    got = N.load(G.gemm(N.store(a, io), N.store(bb, io), None, io, b, f), io)
    exact = a.astype(np.int64) @ bb.astype(np.int64)
    # each tile dot is an integer d: q = d * 2^f (saturated), sum wraps
    bk = G.BLOCK_K[io]
    acc = np.zeros_like(exact)
    for t in range(0, 300, bk):
        d = a[:, t:t + bk].astype(np.int64) @ bb[t:t + bk].astype(np.int64)
        acc += np.clip(d * (1 << f), -(1 << (b - 1)), (1 << (b - 1)) - 1)
    acc = G.wrap_bits(acc, b)
    want = N.round_io((acc.astype(np.float64) * 2.0 ** -f).astype(np.float32), io)
    assert np.array_equal(got, want)
    if b >= 32 and f == 16:
        assert np.array_equal(got, N.round_io(exact.astype(np.float32), io))


def test_accumulator_wraps_and_tiles_saturate():
    # one tile dot of 2^15 saturates Q16.16 int32 (2^31 > qmax)
    a = np.ones((1, 128), np.float32) * 16
    b = np.ones((128, 1), np.float32) * 16
    got = G.gemm(a, b, None, "f32", 32, 16)  # f32 tiles are 64 wide: 2 tiles of 16384
    assert got[0, 0] == np.float32(32768.0 - 2.0 ** -16) * 0 + np.float32((2 * 16384 * 65536 - 2 ** 32) / 65536.0)
    # int64 holds it
    assert G.gemm(a, b, None, "f32", 64, 16)[0, 0] == 32768.0


@pytest.mark.parametrize("io", ["bf16", "f16", "f32"])
def test_ktile_permutation_invariance(io):
    rng = np.random.default_rng(123)
    bk = G.BLOCK_K[io]
    a = N.store(rng.standard_normal((4, 4 * bk)).astype(np.float32), io)
    b = N.store(rng.standard_normal((4 * bk, 4)).astype(np.float32), io)
    perm = np.concatenate([np.arange(t * bk, (t + 1) * bk) for t in (2, 0, 3, 1)])
    c1 = G.gemm(a, b, None, io, 32, 16)
    c2 = G.gemm(a[:, perm], b[perm], None, io, 32, 16)
    assert np.array_equal(np.asarray(c1).view(np.uint8), np.asarray(c2).view(np.uint8))


@pytest.mark.parametrize("io,tol", [("f32", 5e-4), ("f16", 1e-2), ("bf16", 5e-2)])
def test_tolerance_vs_float64(io, tol):
    rng = np.random.default_rng(42)
    a32 = (rng.standard_normal((8, 257)) * 0.5).astype(np.float32)
    b32 = (rng.standard_normal((257, 16)) * 0.5).astype(np.float32)
    bias = rng.standard_normal(16).astype(np.float32)
    a, b = N.store(a32, io), N.store(b32, io)
    got = N.load(G.gemm(a, b, N.store(bias, io), io, 32, 16), io)
    ref = N.load(a, io).astype(np.float64) @ N.load(b, io).astype(np.float64) + N.load(N.store(bias, io), io)
    assert np.allclose(got, N.round_io(ref.astype(np.float32), io), atol=tol, rtol=tol)


def _exact_fixed_gemm(ai, bi, denom, bk, f, b):
    """Independent restatement with Fractions: per-tile exact dot of
    (ai/denom) x (bi/denom), RNE to 2^-f (Fraction round is half-even),
    saturate, wrap-sum."""
    from fractions import Fraction

    M, K = ai.shape
    Nn = bi.shape[1]
    out = np.zeros((M, Nn), np.int64)
    lo, hi = -(1 << (b - 1)), (1 << (b - 1)) - 1
    for m in range(M):
        for n in range(Nn):
            acc = 0
            for t in range(0, K, bk):
                d = sum(int(ai[m, k]) * int(bi[k, n]) for k in range(t, min(K, t + bk)))
                acc += min(max(round(Fraction(d * (1 << f), denom * denom)), lo), hi)
            out[m, n] = acc
    return G.wrap_bits(out, b)


def test_per_tile_rounding_exact_and_planted_mistakes():
    # entries k/16: tile dots are multiples of 1/256 (exact in fp32); at f = 4
    # each tile's RNE (ties included) decides the bits
    rng = np.random.default_rng(3)
    ai = rng.integers(-40, 41, (4, 200))
    bi = rng.integers(-40, 41, (200, 3))
    a, b = (ai / 16).astype(np.float32), (bi / 16).astype(np.float32)
    want = _exact_fixed_gemm(ai, bi, 16, 64, 4, 32)
    got = G.gemm(a, b, None, "f32", 32, 4)
    assert np.array_equal(got, (want * 2.0 ** -4).astype(np.float32))
    # planted mistakes in the oracle must be caught by the same comparison:
    # (1) no per-tile quantisation, (2) truncation instead of RNE,
    # (3) one quantisation of the whole-K sum
    exact = (ai @ bi) / 256.0
    assert not np.array_equal((exact * 16).astype(np.int64), want)
    trunc = sum(np.trunc((ai[:, t:t + 64] @ bi[t:t + 64]) / 16.0) for t in range(0, 200, 64))
    assert not np.array_equal(trunc.astype(np.int64), want)
    once = np.rint(exact * 16).astype(np.int64)
    assert not np.array_equal(once, want)
