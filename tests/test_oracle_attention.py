"""Pin the oracle's paged attention (CPU only).

Tolerance against plain float64 softmax attention (the reference's prefill
test model, fxpr_vllm/_tests/test_prefill.py:22-54, 5e-2), closed forms
(single key -> V on the 2^-f grid; identical keys -> mean of V), page-size and
block-table-permutation invariance (paging is addressing only), exact
whole-tile KV permutation invariance for non-causal attention
(test_prefill.py:246-279), and a planted mistake (dropping the per-tile
quantisation) that the single-key closed form catches.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as A
from oracle import numerics as N


def paged(k, v, ps, perm_seed=None):
    """Contiguous per-token k/v [L, Hkv, D] -> (kv_cache, block_table row)."""
    L, Hkv, D = k.shape
    nb = -(-L // ps)
    kp = np.zeros((nb * ps, Hkv, D), k.dtype)
    vp = np.zeros_like(kp)
    kp[:L], vp[:L] = k, v
    blocks = np.arange(nb)
    if perm_seed is not None:
        blocks = np.random.default_rng(perm_seed).permutation(nb)
    cache = np.zeros((nb, 2, ps, Hkv, D), k.dtype)
    cache[blocks, 0] = kp.reshape(nb, ps, Hkv, D)
    cache[blocks, 1] = vp.reshape(nb, ps, Hkv, D)
    return cache, blocks.astype(np.int32)


def run(q, k, v, ps, io="f32", perm_seed=None, **kw):
    L = k.shape[0]
    cache, bt = paged(N.store(k, io), N.store(v, io), ps, perm_seed)
    T = q.shape[0]
    return N.load(A.unified_attention(N.store(q, io), cache, np.array([0, T], np.int32),
                                      np.array([L], np.int32), bt[None, :], io, **kw), io)


@pytest.mark.parametrize("io,tol", [("f32", 1e-2), ("bf16", 5e-2), ("f16", 5e-2)])
@pytest.mark.parametrize("causal", [True, False])
def test_tolerance_vs_float64(io, tol, causal):
    rng = np.random.default_rng(0)
    L, Hq, Hkv, D = 100, 4, 2, 32
    q = rng.standard_normal((L, Hq, D)).astype(np.float32)
    k = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    got = run(q, k, v, 16, io, is_causal=causal)
    ref = A.attention_reference_fp(N.round_io(q, io), N.round_io(k, io), N.round_io(v, io), [L],
                                   causal, 1 / np.sqrt(D))
    assert np.allclose(got, ref, atol=tol, rtol=tol)


def test_single_key_returns_v_on_the_grid():
    rng = np.random.default_rng(1)
    D = 32
    q = rng.standard_normal((1, 1, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, D)).astype(np.float32)
    v = rng.standard_normal((1, 1, D)).astype(np.float32)
    got = run(q, k, v, 16)
    want = np.rint(v.astype(np.float64) * 65536) / 65536  # one tile, w = 1
    assert np.array_equal(got.astype(np.float64), want)
    # planted mistake: no per-tile quantisation would give v itself
    assert not np.array_equal(got, v)


def test_identical_keys_give_mean_of_v():
    rng = np.random.default_rng(2)
    L, D = 50, 32
    q = rng.standard_normal((1, 1, D)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 1, D)).astype(np.float32), L, axis=0)
    v = rng.standard_normal((L, 1, D)).astype(np.float32)
    got = run(q, k, v, 16, is_causal=False)
    # all weights exactly 1: den = L, wv = RNE(sum v * 2^16) over one tile
    want = np.rint(v.astype(np.float64).sum(0) * 65536) / 65536 / L
    assert np.allclose(got[0], want, atol=1e-6)


def test_paging_is_addressing_only():
    rng = np.random.default_rng(3)
    L, Hq, Hkv, D = 77, 4, 1, 32
    q = rng.standard_normal((5, Hq, D)).astype(np.float32)
    k = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    base = run(q, k, v, 1, "bf16")
    for ps, seed in ((16, None), (16, 5), (32, 7), (1, 9)):
        assert np.array_equal(run(q, k, v, ps, "bf16", perm_seed=seed), base)


@pytest.mark.parametrize("io", ["bf16", "f32"])
def test_whole_tile_kv_permutation_invariance(io):
    rng = np.random.default_rng(7)
    L, D = 192, 32
    q = (rng.standard_normal((L, 2, D)) * 0.5).astype(np.float32)
    k = (rng.standard_normal((L, 2, D)) * 0.5).astype(np.float32)
    v = (rng.standard_normal((L, 2, D)) * 0.5).astype(np.float32)
    base = run(q, k, v, 1, io, is_causal=False)
    idx = np.concatenate([np.arange(t * 64, (t + 1) * 64) for t in (2, 0, 1)])
    assert np.array_equal(run(q, k[idx], v[idx], 1, io, is_causal=False), base)


def test_window_softcap_alibi_tolerance():
    rng = np.random.default_rng(4)
    L, D = 90, 32
    q = rng.standard_normal((L, 2, D)).astype(np.float32)
    k = rng.standard_normal((L, 2, D)).astype(np.float32)
    v = rng.standard_normal((L, 2, D)).astype(np.float32)
    slopes = np.array([0.5, 0.25], np.float32)
    got = run(q, k, v, 16, window_size=20, logit_softcap=5.0,
              alibi_slopes=slopes * np.float32(A.RCP_LN2))
    # float64 model with the same masks / transforms
    s = np.einsum("qhd,khd->hqk", q.astype(np.float64), k.astype(np.float64)) / np.sqrt(D)
    s = 5.0 * np.tanh(s / 5.0)
    pos = np.arange(L)
    s = s + slopes[:, None, None] * (pos[None, None, :] - pos[None, :, None])
    mask = (pos[None, :] <= pos[:, None]) & (pos[None, :] > pos[:, None] - 20)
    s = np.where(mask[None], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("hqk,khd->qhd", p, v.astype(np.float64))
    assert np.allclose(got, ref, atol=2e-3, rtol=2e-3)


# ---------------------------------------------------------------------------
# Key-chunk statistics (the MI355X kernels' algorithm, chunk_keys=CHUNK_KEYS)


@pytest.mark.parametrize("io", ["f32", "bf16"])
@pytest.mark.parametrize("L", [1, 37, 512])
def test_chunked_equals_global_within_one_chunk(io, L):
    # a row whose keys all lie in one chunk: chunk max = row max, and the
    # merge into the empty state is exact, so the bits are the reference's
    rng = np.random.default_rng(L)
    q = rng.standard_normal((3, 4, 32)).astype(np.float32)
    k = rng.standard_normal((L, 2, 32)).astype(np.float32)
    v = rng.standard_normal((L, 2, 32)).astype(np.float32)
    a = run(q, k, v, 16, io, is_causal=False)
    b = run(q, k, v, 16, io, is_causal=False, chunk_keys=A.CHUNK_KEYS)
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("io,tol", [("f32", 1e-2), ("bf16", 5e-2)])
@pytest.mark.parametrize("causal", [True, False])
def test_chunked_tolerance_vs_float64(io, tol, causal):
    # 2100 keys = 5 chunks; a ramp in the keys makes the chunk maxima differ
    # by several units of log2, so every merge rescales both sides
    rng = np.random.default_rng(5)
    L, Hq, Hkv, D = 2100, 2, 1, 32
    q = rng.standard_normal((4, Hq, D)).astype(np.float32)
    k = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    k += (np.linspace(-1.0, 1.0, L)[:, None, None] * q[:1, :1, :].mean(axis=1, keepdims=True)).astype(np.float32)
    v = rng.standard_normal((L, Hkv, D)).astype(np.float32)
    got = run(q, k, v, 16, io, is_causal=causal, chunk_keys=A.CHUNK_KEYS)
    # q rows are the last 4 positions of the sequence
    qq = np.zeros((L, Hq, D), np.float32)
    qq[-4:] = q
    ref = A.attention_reference_fp(N.round_io(qq, io), N.round_io(k, io), N.round_io(v, io), [L],
                                   causal, 1 / np.sqrt(D))[-4:]
    assert np.allclose(got, ref, atol=tol, rtol=tol)
    glob = run(q, k, v, 16, io, is_causal=causal)
    assert np.allclose(got, glob, atol=tol, rtol=tol)


def test_merge_chunk_closed_forms():
    # equal maxima: plain integer sums; a chunk 1 below the running max is
    # halved (RNE on the fixed-point grid); a -inf chunk changes nothing
    st = (np.array([2.0, 2.0, 2.0], np.float32), np.array([100, 101, 7], np.int64),
          np.array([[10, -3], [11, 5], [1, 1]], np.int64))
    m_c = np.array([2.0, 1.0, -np.inf], np.float32)
    M, D, W = A.merge_chunk(st, m_c, np.array([50, 51, 9]), np.array([[4, 4], [3, -5], [9, 9]]), 32)
    assert M.tolist() == [2.0, 2.0, 2.0]
    assert D.tolist() == [150, 101 + 26, 7]          # 51/2 = 25.5 -> 26 (even)
    assert W.tolist() == [[14, 1], [11 + 2, 5 - 2], [1, 1]]  # 3/2 -> 2, -5/2 -> -2
    # a chunk 1 above: the running state is halved instead
    M, D, W = A.merge_chunk(st, np.array([3.0, 3.0, 3.0], np.float32), np.array([8, 8, 8]),
                            np.zeros((3, 2), np.int64), 32)
    assert M.tolist() == [3.0, 3.0, 3.0] and D.tolist() == [58, 58, 12]  # 50+8, 50.5->50 +8, 3.5->4 +8


def test_planted_merge_mistake_is_caught():
    # swapping the two rescale factors (a plausible slip) breaks the float64
    # tolerance on rows whose chunk maxima differ
    rng = np.random.default_rng(5)
    L, D = 1500, 32
    q = rng.standard_normal((2, 2, D)).astype(np.float32)
    k = rng.standard_normal((L, 1, D)).astype(np.float32) * np.linspace(0.2, 2.0, L)[:, None, None].astype(np.float32)
    v = rng.standard_normal((L, 1, D)).astype(np.float32)
    good = run(q, k, v, 16, "f32", is_causal=False, chunk_keys=A.CHUNK_KEYS)
    orig = A.merge_chunk

    def swapped(state, m_c, den_c, wv_c, int_bits):
        M, Dd, W = state
        live = np.isfinite(m_c)
        Mn = np.where(live, np.maximum(M, m_c), M).astype(np.float32)
        with np.errstate(invalid="ignore", over="ignore"):
            fb = np.nan_to_num(np.exp2((M - Mn).astype(np.float64))).astype(np.float32)
            fa = np.nan_to_num(np.exp2((m_c - Mn).astype(np.float64))).astype(np.float32)
        Dn = A._rescale(Dd, fa, int_bits) + A._rescale(den_c, fb, int_bits)
        Wn = A._rescale(W, fa[:, None], int_bits) + A._rescale(wv_c, fb[:, None], int_bits)
        return (np.where(live, Mn, M).astype(np.float32), np.where(live, Dn, Dd), np.where(live[:, None], Wn, W))

    A.merge_chunk = swapped
    try:
        bad = run(q, k, v, 16, "f32", is_causal=False, chunk_keys=A.CHUNK_KEYS)
    finally:
        A.merge_chunk = orig
    ref = A.attention_reference_fp(np.concatenate([np.zeros((L - 2, 2, D), np.float32), q]), k, v, [L], False,
                                   1 / np.sqrt(D))[-2:]
    assert np.allclose(good, ref, atol=1e-2, rtol=1e-2)
    assert not np.allclose(bad, ref, atol=1e-2, rtol=1e-2)
