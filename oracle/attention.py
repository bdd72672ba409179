"""Unified paged attention with fixed-point cross-tile reductions, in numpy."""

from __future__ import annotations

import math

import numpy as np

from .numerics import F32, fixed_to_f32, load, rne_sat, round_io, store
from .gemm import wrap_bits

RCP_LN2 = 1.4426950408889634
BLOCK_N = {"bf16": 64, "f16": 64, "f32": 32}


CHUNK_KEYS = 512  # key chunk of the MI355X kernels' softmax statistics


def _rescale(x, f, int_bits):
    """RNE(fl64(x) * fl64(f)), saturated to int_bits: an int_bits fixed-point
    value (wrapped to int_bits first) scaled by f <= 1."""
    x = wrap_bits(np.asarray(x, np.int64), int_bits).astype(np.float64)
    r = np.rint(x * np.asarray(f, np.float32).astype(np.float64))
    lim = 2.0 ** (int_bits - 1)
    r = np.where(r >= lim, lim - 1, np.where(r < -lim, -lim, r))
    return r.astype(np.int64)


def merge_chunk(state, m_c, den_c, wv_c, int_bits):
    """Fold one key chunk's statistics into a row's running state, in
    fixed point: state (M, D, W) with M the largest chunk maximum so far.

    M' = max(M, m_c); D' = wrap(resc(D, 2^(M - M')) + resc(den_c, 2^(m_c - M')))
    and W' likewise, resc = _rescale, the powers of two formed in fp32. Chunks
    whose m_c is -inf (no valid key for the row) leave the state unchanged.
    This build's semantics (the MI355X kernels' key chunks); the reference
    normalises every key against the row's global maximum instead."""
    M, D, W = state
    live = np.isfinite(m_c)
    Mn = np.where(live, np.maximum(M, m_c), M).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        fa = np.where(live, np.exp2((M - Mn).astype(np.float64)), 1.0).astype(np.float32)
        fb = np.where(live, np.exp2((m_c - Mn).astype(np.float64)), 0.0).astype(np.float32)
    fa = np.where(np.isnan(fa), 0.0, fa).astype(np.float32)
    fb = np.where(np.isnan(fb), 0.0, fb).astype(np.float32)
    Dn = wrap_bits(_rescale(D, fa, int_bits) + _rescale(den_c, fb, int_bits), int_bits)
    Wn = wrap_bits(_rescale(W, fa[:, None], int_bits) + _rescale(wv_c, fb[:, None], int_bits), int_bits)
    return (np.where(live, Mn, M).astype(np.float32), np.where(live, Dn, D),
            np.where(live[:, None], Wn, W))


def unified_attention(q, kv_cache, query_start_loc, seq_lens, block_table, io, *,
                      is_causal=True, softmax_scale=None, alibi_slopes=None,
                      int_bits=32, frac_bits=16, logit_softcap=0.0, window_size=0,
                      chunk_keys=None):
    """Returns o [T, Hq, D] (storage of `io`).

    Follows fxpr_vllm/_triton/attention.py: scores scaled into log2 space
    (:748-750, :114), softcap softcap*tanh(s/softcap) (:115-116), ALiBi
    slope*(n - qpos) (:117-120), causal / window / sequence masks (:208-215,
    :249-254), exact row max over all keys (:233-257, :563-577), w = exp2(s - m)
    (:285), denominator = integer sum of per-key float_to_fixed(w) (:286),
    weighted V = integer sum over key tiles of float_to_fixed(fp32 dot of
    IO(w) and V over the tile) (:287-290), o = IO(num / max(den, 1e-6))
    (:292-301); paged addressing block_table[r, n // page], slot n % page
    (:238-243).
    Build choice: key tiles are aligned to absolute key positions
    (multiples of BLOCK_N = 64 for bf16/f16, 32 for f32); the reference
    aligns them at the q-block's window start, which only differs when a
    sliding window is set.
    Parity unpinned at the bit level: the fp32 dot orders (tl.dot / MFMA /
    here float64 rounded once) and the reference's libdevice exp2 / tanh.
    Pinned by tolerance, invariances and closed forms (tests).

    chunk_keys=None is the reference's algorithm (one maximum per row).
    chunk_keys=CHUNK_KEYS is the MI355X kernels' algorithm: keys in absolute
    chunks of chunk_keys, each chunk's weights w = exp2(s - m_c) taken against
    the chunk's own maximum m_c, and the per-chunk integer (den, wv) folded in
    ascending chunk order by merge_chunk. A row whose keys all lie in one
    chunk gets the reference's bits exactly.
    """
    qf = load(np.asarray(q), io).astype(np.float64)
    kv = load(np.asarray(kv_cache), io)
    T, Hq, D = qf.shape
    NB, _, ps, Hkv, _ = kv.shape
    G = Hq // Hkv
    bn = BLOCK_N[io]
    qsl = np.asarray(query_start_loc).astype(np.int64)
    sl = np.asarray(seq_lens).astype(np.int64)
    bt = np.asarray(block_table).astype(np.int64)
    ss = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    ss_log2 = F32(float(ss) * RCP_LN2)
    cap = F32(float(logit_softcap) * RCP_LN2) if logit_softcap > 0 else None
    scale = F32(2.0 ** frac_bits)
    out = np.zeros((T, Hq, D), np.float32)
    for r in range(len(sl)):
        q0, q1 = int(qsl[r]), int(qsl[r + 1])
        qlen, L = q1 - q0, int(sl[r])
        if qlen == 0:
            continue
        ctx = L - qlen
        nblk = -(-L // ps)
        blocks = bt[r, :nblk]
        K = kv[blocks, 0].reshape(nblk * ps, Hkv, D)[:L].astype(np.float64)
        V = kv[blocks, 1].reshape(nblk * ps, Hkv, D)[:L].astype(np.float64)
        ntiles = -(-L // bn)
        Lp = ntiles * bn
        qpos = ctx + np.arange(qlen)
        n = np.arange(L)
        kend = np.minimum(L, qpos + 1) if is_causal else np.full(qlen, L)
        kstart = np.maximum(0, qpos - window_size + 1) if window_size > 0 else np.zeros(qlen, np.int64)
        valid = (n[None, :] >= kstart[:, None]) & (n[None, :] < kend[:, None])
        for h in range(Hq):
            g = h // G
            s = (qf[q0:q1, h, :] @ K[:, g, :].T).astype(np.float32) * ss_log2
            if cap is not None:
                s = (cap * np.tanh((s / cap).astype(np.float64))).astype(np.float32)
            if alibi_slopes is not None:
                s = s + F32(np.asarray(alibi_slopes, np.float32)[h]) * (n[None, :] - qpos[:, None]).astype(np.float32)
            s = np.where(valid, s, F32(-np.inf)).astype(np.float32)
            vv = np.zeros((Lp, D))
            vv[:L] = V[:, g, :]

            def stats(k0, k1):
                """(max, den, wv) of keys [k0, k1) (tile-aligned), weights
                against that range's own row maxima."""
                sc = np.full((qlen, k1 - k0), F32(-np.inf), np.float32)
                sc[:, : max(0, min(L, k1) - k0)] = s[:, k0:min(L, k1)]
                m_raw = sc.max(axis=1)
                m = np.where(np.isfinite(m_raw), m_raw, F32(0.0))
                with np.errstate(invalid="ignore", over="ignore"):
                    w = np.exp2((sc - m[:, None]).astype(np.float64)).astype(np.float32)
                    den = wrap_bits(rne_sat(w * scale, int_bits).sum(axis=1), int_bits)
                p = round_io(w, io).astype(np.float64)
                nt = (k1 - k0) // bn
                pv = np.einsum("qtn,tnd->qtd", p.reshape(qlen, nt, bn),
                               vv[k0:k1].reshape(nt, bn, D)).astype(np.float32)
                with np.errstate(invalid="ignore", over="ignore"):
                    wv = wrap_bits(rne_sat(pv * scale, int_bits).sum(axis=1), int_bits)
                return m_raw, den, wv

            if chunk_keys is None:
                _, den, wv = stats(0, Lp)
            else:
                state = (np.full(qlen, F32(-np.inf), np.float32), np.zeros(qlen, np.int64),
                         np.zeros((qlen, D), np.int64))
                for k0 in range(0, Lp, chunk_keys):
                    state = merge_chunk(state, *stats(k0, min(Lp, k0 + chunk_keys)), int_bits)
                _, den, wv = state
            den_f = np.maximum(fixed_to_f32(den, frac_bits), F32(1e-6))
            out[q0:q1, h, :] = fixed_to_f32(wv, frac_bits) / den_f[:, None]
    return store(out, io)


def attention_reference_fp(q, k, v, seq_lens_list, is_causal, sm_scale):
    """Plain float64 softmax attention over contiguous per-request q/k/v, the
    model the reference's prefill tests compare against
    (fxpr_vllm/_tests/test_prefill.py:22-54)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T, Hq, D = q.shape
    G = Hq // k.shape[1]
    o = np.zeros_like(q)
    start = 0
    for L in seq_lens_list:
        for h in range(Hq):
            s = q[start:start + L, h] @ k[start:start + L, h // G].T * sm_scale
            if is_causal:
                s = np.where(np.triu(np.ones((L, L), bool), 1), -1e30, s)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            o[start:start + L, h] = p @ v[start:start + L, h // G]
        start += L
    return o
