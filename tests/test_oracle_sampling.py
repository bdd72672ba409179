"""Pin the oracle's greedy sampler (CPU only).

The order is checked against an independent Python sort on (value, index)
tuples with the stated rules (NaN first, -0 == +0, ties to the lower index),
the sampled token against numpy.argmax (first maximum, NaN wins), and the
log-probabilities against the log-softmax oracle. Two plausible mistakes
(tie to the higher index, a sign-blind float order) are planted and caught.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import numerics as N
from oracle import rows as R
from oracle import sampling as S


def brute_order(row):
    def key(j):
        v = float(row[j])
        if math.isnan(v):
            return (0, 0.0, j)           # NaN ranks first, then by index
        return (1, -(v + 0.0), j)        # larger first (-0 == +0), then lower index
    return sorted(range(len(row)), key=key)


def tie_rows(seed=0, V=257):
    rng = np.random.default_rng(seed)
    x = rng.integers(-4, 5, (6, V)).astype(np.float32)   # many ties
    x[1, 7] = np.nan
    x[1, 200] = np.nan
    x[2] = 0.0
    x[2, ::3] = -0.0
    x[3, 10] = np.inf
    x[3, 11] = np.inf
    x[4] = -np.inf
    x[5] = rng.standard_normal(V).astype(np.float32) * -3
    return x


@pytest.mark.parametrize("k", [0, 1, 5, 64])
def test_order_matches_brute_force(k):
    x = tie_rows()
    ids, lp, top, top_lp = S.sample_greedy(x, "f32", k, 32, 16)
    y = R.log_softmax(x, "f32", "f32", 32, 16)
    for r in range(x.shape[0]):
        want = brute_order(x[r])
        assert ids[r] == want[0]
        assert list(top[r]) == want[:k]
        assert np.array_equal(top_lp[r].view(np.uint32), y[r, want[:k]].view(np.uint32))
        assert lp[r].view(np.uint32) == y[r, want[0]].view(np.uint32)


def test_sampled_token_is_numpy_argmax():
    rng = np.random.default_rng(1)
    x = np.round(rng.standard_normal((20, 1000)) * 3, 1).astype(np.float32)
    x[3, 500] = np.nan
    ids, _, _, _ = S.sample_greedy(x, "f32", 0, 32, 16)
    assert np.array_equal(ids, np.argmax(x, axis=1))


def test_bf16_input():
    rng = np.random.default_rng(2)
    x = N.store((rng.standard_normal((4, 300)) * 4).astype(np.float32), "bf16")
    ids, _, top, _ = S.sample_greedy(x, "bf16", 8, 64, 32)
    xf = N.load(x, "bf16")
    for r in range(4):
        assert list(top[r]) == brute_order(xf[r])[:8]


def test_planted_mistakes_are_caught(monkeypatch):
    x = tie_rows(seed=3)
    real = S.value_order

    def differs():
        ids, _, top, _ = S.sample_greedy(x, "f32", 16, 32, 16)
        return any(list(top[r]) != brute_order(x[r])[:16] for r in range(x.shape[0]))

    assert not differs()
    # a float order that ignores the sign bit
    monkeypatch.setattr(S, "value_order", lambda xf: np.asarray(xf, np.float32).view(np.uint32))
    assert differs()
    monkeypatch.setattr(S, "value_order", real)
    # ties to the higher index
    monkeypatch.setattr(S.np, "uint64", np.uint64)
    orig = S.sample_greedy

    def hi_tie(xx, io, k, b, f):
        xf = N.load(np.asarray(xx), io)
        keys = (real(xf).astype(np.uint64) << np.uint64(32)) | np.arange(xf.shape[1], dtype=np.uint64)[None, :]
        order = np.argsort(keys, axis=1)[:, ::-1]
        return order[:, 0], None, order[:, :k], None

    monkeypatch.setattr(S, "sample_greedy", hi_tie)
    assert differs()
    monkeypatch.setattr(S, "sample_greedy", orig)
