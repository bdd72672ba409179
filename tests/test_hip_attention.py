"""GPU parity: paged attention (HIP/MFMA) vs the oracle and the reference's
decode / prefill tests (fxpr_vllm/_tests/test_decode.py, test_prefill.py),
restated.

Within 1e-2 of the oracle on seeded data (the
kernels' 512-key chunk statistics, and the reference's one-maximum-per-row
algorithm on the same data); bitwise
identical across KV split counts, batch composition, the decode vs prefill
path, run-to-run, and whole-tile KV permutations (non-causal).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fxpr_vllm  # noqa: F401
from oracle import attention as A
from tests._util import IO_NAME, close_report, from_np, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
RCP_LN2 = 1.4426950408889634


def attend(q, kv, qsl, sl, bt, max_q, splits, *, causal=True, scale=None, alibi=None,
           bits=32, frac=16, softcap=0.0, window=0):
    o = torch.empty_like(q)
    torch.ops.fxpr.unified_attention_fxp(q, kv, o, qsl, sl, bt, int(max_q), alibi, bool(causal),
                                         scale, bits, frac, float(softcap), int(window), int(splits))
    return o


def oracle(q, kv, qsl, sl, bt, *, causal=True, scale=None, alibi=None, bits=32, frac=16,
           softcap=0.0, window=0, chunk_keys=A.CHUNK_KEYS):
    """The kernels' algorithm (512-key chunk statistics) by default;
    chunk_keys=None is the reference's (one maximum per row)."""
    io = IO_NAME[q.dtype]
    out = A.unified_attention(to_np(q), to_np(kv), qsl.cpu().numpy(), sl.cpu().numpy(), bt.cpu().numpy(),
                              io, is_causal=causal, softmax_scale=scale,
                              alibi_slopes=None if alibi is None else alibi.cpu().numpy(),
                              int_bits=bits, frac_bits=frac, logit_softcap=softcap, window_size=window,
                              chunk_keys=chunk_keys)
    return from_np(out, q.dtype)


def decode_case(batch, hq, hkv, d, ctx_lo, ctx_hi, ps, dtype, seed=0, pool_extra=7):
    g = torch.Generator("cpu").manual_seed(seed)
    sl = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=g, dtype=torch.int32)
    maxb = int((sl.max().item() + ps - 1) // ps)
    nb = batch * maxb + pool_extra
    perm = torch.randperm(nb, generator=g)[: batch * maxb].to(torch.int32)
    bt = perm.reshape(batch, maxb)
    q = torch.randn(batch, hq, d, generator=g).to(dtype)
    kv = torch.randn(nb, 2, ps, hkv, d, generator=g).to(dtype)
    qsl = torch.arange(batch + 1, dtype=torch.int32)
    return q.to(DEV), kv.to(DEV), qsl.to(DEV), sl.to(DEV), bt.to(DEV)


def prefill_case(seq_lens, hq, hkv, d, dtype, seed=42, scale=1.0):
    """Contiguous q/k/v into a page-size-1 cache with a per-request block
    table, like the reference helper prefill_fxp_test
    (fxpr_vllm/_tests/fixed_point_helpers.py:80-145)."""
    g = torch.Generator("cpu").manual_seed(seed)
    T = sum(seq_lens)
    q = (torch.randn(T, hq, d, generator=g) * scale).to(dtype)
    k = (torch.randn(T, hkv, d, generator=g) * scale).to(dtype)
    v = (torch.randn(T, hkv, d, generator=g) * scale).to(dtype)
    kv = torch.empty(T, 2, 1, hkv, d, dtype=dtype)
    kv[:, 0, 0] = k
    kv[:, 1, 0] = v
    maxl = max(seq_lens)
    bt = torch.zeros(len(seq_lens), maxl, dtype=torch.int32)
    start = 0
    for r, L in enumerate(seq_lens):
        bt[r, :L] = torch.arange(start, start + L, dtype=torch.int32)
        start += L
    qsl = torch.tensor([0] + list(np.cumsum(seq_lens)), dtype=torch.int32)
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    return (q.to(DEV), kv.to(DEV), qsl.to(DEV), sl.to(DEV), bt.to(DEV)), (q, k, v)


def close(got, want, tol=1e-2):
    """Per element |got - want| <= tol * |want| + 1e-2 * RMS(want).

    The floor covers outputs near zero: every weight P is rounded to the I/O
    type before the weighted-V product (the reference's IO(w),
    fxpr_vllm/_triton/attention.py:287), so two orders of the same softmax
    (512-key chunk maxima vs one maximum per row, or NVIDIA vs MFMA) differ by
    bf16 rounding noise of about 2^-9 * RMS(V) / sqrt(keys) per element."""
    report = close_report(got, want, rtol=tol, atol_rms=1e-2)
    assert not report, report
    return True


# --------------------------------------------------------------------------
# decode


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_gqa_vs_oracle_and_split_invariance(dtype):
    q, kv, qsl, sl, bt = decode_case(6, 32, 8, 128, 100, 1500, 16, dtype)
    ref = attend(q, kv, qsl, sl, bt, 1, 1)
    for s in (2, 3, 4, 8, 16, 0):
        assert torch.equal(attend(q, kv, qsl, sl, bt, 1, s), ref), s
    assert close(ref, oracle(q, kv, qsl, sl, bt))
    # contexts up to 1500 keys span 3 chunks: the reference's global-maximum
    # algorithm agrees within the same tolerance
    assert close(ref, oracle(q, kv, qsl, sl, bt, chunk_keys=None))


@pytest.mark.parametrize("bits,frac", [(64, 32), (64, 16), (16, 8)])
def test_decode_fixed_point_formats(bits, frac):
    q, kv, qsl, sl, bt = decode_case(4, 8, 2, 64, 50, 700, 16, torch.bfloat16, seed=3)
    ref = attend(q, kv, qsl, sl, bt, 1, 1, bits=bits, frac=frac)
    assert torch.equal(attend(q, kv, qsl, sl, bt, 1, 5, bits=bits, frac=frac), ref)
    tol = 1e-2 if bits > 16 else 5e-2  # Q8 in int16 is coarse by design
    assert close(ref, oracle(q, kv, qsl, sl, bt, bits=bits, frac=frac), tol)


@pytest.mark.parametrize("d", [64, 96, 256])
def test_decode_head_dims(d):
    q, kv, qsl, sl, bt = decode_case(3, 8, 8, d, 10, 300, 16, torch.bfloat16, seed=d)
    ref = attend(q, kv, qsl, sl, bt, 1, 1)
    assert torch.equal(attend(q, kv, qsl, sl, bt, 1, 4), ref)
    assert close(ref, oracle(q, kv, qsl, sl, bt))


# restated: fxpr_vllm/_tests/test_decode.py (4 q heads, 2 kv heads, d 32, page 16,
# identity block table)

def _ref_decode_inputs(seq_lens, nbps, dtype):
    g = torch.Generator("cpu").manual_seed(2026)
    R = len(seq_lens)
    q = torch.randn(R, 4, 32, generator=g).to(dtype)
    kv = torch.randn(R * nbps, 2, 16, 2, 32, generator=g).to(dtype)
    return (q.to(DEV), kv.to(DEV), torch.arange(R + 1, dtype=torch.int32, device=DEV),
            torch.tensor(seq_lens, dtype=torch.int32, device=DEV),
            torch.arange(R * nbps, dtype=torch.int32, device=DEV).reshape(R, nbps))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("splits", [1, 2, 4, 8])
def test_reference_decode_invariant_across_kv_splits(dtype, splits):
    args = _ref_decode_inputs([160, 96], 10, dtype)
    o1 = attend(*args, 1, 1, scale=1 / math.sqrt(32))
    assert torch.equal(o1, attend(*args, 1, splits, scale=1 / math.sqrt(32)))


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_decode_deterministic_and_native_dtype(dtype):
    args = _ref_decode_inputs([128, 192, 64], 12, dtype)
    first = attend(*args, 1, 4, scale=1 / math.sqrt(32))
    for _ in range(4):
        assert torch.equal(first, attend(*args, 1, 4, scale=1 / math.sqrt(32)))
    args = _ref_decode_inputs([48, 32], 3, dtype)
    o = attend(*args, 1, 4, scale=1 / math.sqrt(32))
    assert o.dtype == dtype and o.shape == args[0].shape and torch.isfinite(o.float()).all()


# --------------------------------------------------------------------------
# prefill


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch,causal", [(1, True), (2, True), (1, False)])
def test_reference_prefill_correctness(dtype, batch, causal):
    # fxpr_vllm/_tests/test_prefill.py:97-137
    lens = [32] * batch
    args, (q, k, v) = prefill_case(lens, 2, 2, 32, dtype)
    o = attend(*args, 32, 1, causal=causal, scale=1 / math.sqrt(32))
    ref = A.attention_reference_fp(q.float().numpy(), k.float().numpy(), v.float().numpy(), lens, causal,
                                   1 / math.sqrt(32))
    assert np.allclose(o.float().cpu().numpy(), ref, atol=5e-2, rtol=5e-2)


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_prefill_variable_seq_lens_and_oracle(dtype):
    # fxpr_vllm/_tests/test_prefill.py:140-158 plus the oracle at 1e-2
    lens = [70, 128, 100]
    args, (q, k, v) = prefill_case(lens, 2, 2, 32, dtype, seed=99)
    o = attend(*args, max(lens), 1, scale=1 / math.sqrt(32))
    ref = A.attention_reference_fp(q.float().numpy(), k.float().numpy(), v.float().numpy(), lens, True,
                                   1 / math.sqrt(32))
    assert np.allclose(o.float().cpu().numpy(), ref, atol=5e-2, rtol=5e-2)
    assert close(o, oracle(*args, scale=1 / math.sqrt(32)))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("splits", [1, 2, 4, 8])
def test_reference_prefill_invariant_across_kv_splits(dtype, splits):
    # fxpr_vllm/_tests/test_prefill.py:161-184
    args, _ = prefill_case([96, 64], 2, 2, 32, dtype, seed=5)
    o1 = attend(*args, 96, 1, scale=1 / math.sqrt(32))
    assert torch.equal(o1, attend(*args, 96, splits, scale=1 / math.sqrt(32)))


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_prefill_tile_permutation_invariance(dtype):
    # fxpr_vllm/_tests/test_prefill.py:246-279: permuting whole 64-key tiles
    L = 192
    g = torch.Generator("cpu").manual_seed(7)
    q = torch.randn(L, 2, 32, generator=g) * 0.5
    k = torch.randn(L, 2, 32, generator=g) * 0.5
    v = torch.randn(L, 2, 32, generator=g) * 0.5
    idx = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in (2, 0, 1)])

    def run(kk, vv):
        kv = torch.empty(L, 2, 1, 2, 32)
        kv[:, 0, 0], kv[:, 1, 0] = kk, vv
        bt = torch.arange(L, dtype=torch.int32).reshape(1, L)
        qsl = torch.tensor([0, L], dtype=torch.int32)
        sl = torch.tensor([L], dtype=torch.int32)
        return attend(q.to(dtype).to(DEV), kv.to(dtype).to(DEV), qsl.to(DEV), sl.to(DEV), bt.to(DEV), L, 1,
                      causal=False, scale=1 / math.sqrt(32))

    assert torch.equal(run(k, v), run(k[idx], v[idx]))


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_prefill_deterministic(dtype):
    args, _ = prefill_case([32], 2, 2, 32, dtype, seed=77)
    r0 = attend(*args, 32, 1, scale=1 / math.sqrt(32))
    for _ in range(4):
        assert torch.equal(r0, attend(*args, 32, 1, scale=1 / math.sqrt(32)))


# --------------------------------------------------------------------------
# batch composition and path invariance


def test_batch_composition_and_decode_prefill_paths_are_bitwise_identical():
    dtype = torch.bfloat16
    g = torch.Generator("cpu").manual_seed(11)
    hq, hkv, d, ps = 8, 2, 128, 16
    lens = [300, 77, 1000]
    nb = sum((L + ps - 1) // ps for L in lens) + 3
    kv = torch.randn(nb, 2, ps, hkv, d, generator=g).to(dtype).to(DEV)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    tables, off = [], 0
    for L in lens:
        n = (L + ps - 1) // ps
        tables.append(perm[off:off + n])
        off += n
    qs = [torch.randn(L, hq, d, generator=g).to(dtype).to(DEV) for L in lens]

    def batch(members):
        """members: list of (request index, q_len); queries are the last
        q_len tokens of that request."""
        q = torch.cat([qs[i][lens[i] - ql:] for i, ql in members])
        maxb = max(len(tables[i]) for i, _ in members)
        bt = torch.zeros(len(members), maxb, dtype=torch.int32)
        for j, (i, _) in enumerate(members):
            bt[j, :len(tables[i])] = tables[i]
        qsl = torch.tensor([0] + list(np.cumsum([ql for _, ql in members])), dtype=torch.int32)
        sl = torch.tensor([lens[i] for i, _ in members], dtype=torch.int32)
        maxq = max(ql for _, ql in members)
        return attend(q, kv, qsl.to(DEV), sl.to(DEV), bt.to(DEV), maxq, 0).cpu(), qsl

    full, _ = batch([(0, lens[0])])          # request 0 prefilled entirely
    dec, _ = batch([(0, 1)])                 # request 0's last token as a decode
    assert torch.equal(dec[0], full[-1])
    mixed, qsl = batch([(2, 1), (0, 5), (1, 77)])   # decode + partial prefill + prefill
    assert torch.equal(mixed[1:6], full[-5:])
    alone2, _ = batch([(2, 1)])
    assert torch.equal(mixed[0], alone2[0])
    big, _ = batch([(1, 1), (2, 1), (0, 1)])
    assert torch.equal(big[2], dec[0]) and torch.equal(big[1], alone2[0])


# --------------------------------------------------------------------------
# features


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_alibi_softcap_window_vs_oracle(dtype):
    args, _ = prefill_case([90, 40], 4, 2, 64, dtype, seed=4)
    slopes = torch.tensor([0.5, 0.25, 0.125, 0.0625], dtype=torch.float32) * RCP_LN2
    kw = dict(alibi=slopes.to(DEV), softcap=5.0, window=20)
    o = attend(*args, 90, 1, **kw)
    assert torch.equal(o, attend(*args, 90, 3, **kw))
    assert close(o, oracle(*args, alibi=slopes, softcap=5.0, window=20))


def test_attention_errors_and_empty():
    q, kv, qsl, sl, bt = decode_case(2, 4, 2, 32, 10, 40, 16, torch.bfloat16)
    with pytest.raises(TypeError):
        attend(q.float(), kv, qsl, sl, bt, 1, 1)
    with pytest.raises(TypeError):
        attend(q, kv, qsl.long(), sl, bt, 1, 1)
    with pytest.raises(ValueError):
        attend(q, kv[:, 0], qsl, sl, bt, 1, 1)
    with pytest.raises(ValueError):
        attend(q, kv, qsl, sl, bt, 1, -1)
    o = torch.full_like(q, 7.0)
    torch.ops.fxpr.unified_attention_fxp(q, kv, o, qsl[:1], sl[:0], bt[:0], 1, None, True, None, 32, 16,
                                         0.0, 0, 1)
    assert torch.all(o == 7.0)


def test_config4_decode_full_shape_properties():
    # the bench shape: batch 64, 32/8 heads, d 128, ctx U[512, 8192], page 16,
    # block table from a permutation of a 2^16-block pool; KV generated on
    # the device. Split invariance for {1, 2, 4, 8, 16} and auto; an oracle
    # check on three requests.
    g = torch.Generator("cpu").manual_seed(0)
    B, hq, hkv, d, ps, pool = 64, 32, 8, 128, 16, 1 << 16
    sl = torch.randint(512, 8193, (B,), generator=g, dtype=torch.int32)
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    bt = perm[: B * 512].reshape(B, 512)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16).to(DEV)
    gd = torch.Generator(DEV).manual_seed(1)
    kv = torch.randn(pool, 2, ps, hkv, d, generator=gd, device=DEV, dtype=torch.bfloat16)
    qsl = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    sl_d, bt_d = sl.to(DEV), bt.to(DEV)
    ref = attend(q, kv, qsl, sl_d, bt_d, 1, 1)
    for s in (2, 4, 8, 16, 0):
        assert torch.equal(attend(q, kv, qsl, sl_d, bt_d, 1, s), ref), s
    longest = int(torch.argmax(sl))
    for r in (0, 17, longest):
        nblk = (int(sl[r]) + ps - 1) // ps
        blocks = bt[r, :nblk].long()
        sub_kv = kv[blocks.to(DEV)].cpu()
        sub_bt = torch.arange(nblk, dtype=torch.int32).reshape(1, nblk)
        sub = (q[r:r + 1].cpu(), sub_kv, torch.tensor([0, 1], dtype=torch.int32), sl[r:r + 1], sub_bt)
        # the kernels' algorithm (512-key chunks) and the reference's (one
        # maximum per row), up to the longest context (16 chunks)
        assert close(ref[r:r + 1], oracle(*sub))
        assert close(ref[r:r + 1], oracle(*sub, chunk_keys=None))
    assert int(sl[longest]) > 7680  # 16 chunks of 512 keys


@pytest.mark.parametrize("R", [63, 200, 256, 257])
def test_decode_request_order_many_requests_with_ties(R):
    # Unsplit and multi-chunk split launches dispatch the requests longest
    # first (ties by index; up to 256 requests), the one-chunk splits of the
    # automatic plan in launch order. The order must be a permutation: every
    # row written once (outputs start as NaN) and the bits of every split
    # count equal; rows of a short, a tied and the longest request against
    # the oracle.
    g = torch.Generator("cpu").manual_seed(R)
    hq, hkv, d, ps = 8, 2, 128, 16
    choices = torch.tensor([1, 17, 511, 512, 513, 1500, 2600], dtype=torch.int32)
    sl = choices[torch.randint(0, len(choices), (R,), generator=g)]
    maxb = (int(sl.max()) + ps - 1) // ps
    pool = R * maxb
    bt = torch.randperm(pool, generator=g).to(torch.int32).reshape(R, maxb)
    q = torch.randn(R, hq, d, generator=g).to(torch.bfloat16).to(DEV)
    gd = torch.Generator(DEV).manual_seed(2)
    kv = torch.randn(pool, 2, ps, hkv, d, generator=gd, device=DEV, dtype=torch.bfloat16)
    qsl = torch.arange(R + 1, dtype=torch.int32, device=DEV)
    sl_d, bt_d = sl.to(DEV), bt.to(DEV)

    def run(splits):
        o = torch.full_like(q, float("nan"))
        torch.ops.fxpr.unified_attention_fxp(q, kv, o, qsl, sl_d, bt_d, 1, None, True, None, 32, 16, 0.0, 0,
                                             splits)
        assert not torch.isnan(o).any(), splits
        return o

    ref = run(0)
    for s in (1, 2, 3):
        assert torch.equal(run(s), ref), s
    longest = int(torch.argmax(sl))
    tied = [i for i in range(R) if int(sl[i]) == int(sl[longest]) and i != longest]
    for r in [int(torch.argmin(sl)), longest] + tied[:1]:
        nblk = (int(sl[r]) + ps - 1) // ps
        sub_kv = kv[bt[r, :nblk].long().to(DEV)].cpu()
        sub_bt = torch.arange(nblk, dtype=torch.int32).reshape(1, nblk)
        sub = (q[r:r + 1].cpu(), sub_kv, torch.tensor([0, 1], dtype=torch.int32), sl[r:r + 1], sub_bt)
        assert close(ref[r:r + 1], oracle(*sub))


# --------------------------------------------------------------------------
# 128-row prefill workgroups (16-bit inputs, Q <= 32-bit accumulators,
# head_dim <= 128, one split, max_query_len * group >= 113) against the
# generic kernel's split path: the bits must not depend on which runs


def _prefix_case(q_lens, ctxs, hq, hkv, d, ps, dtype, seed):
    """Requests with a cached prefix of ctxs[i] keys and q_lens[i] new tokens,
    pages shuffled over one pool."""
    g = torch.Generator("cpu").manual_seed(seed)
    sls = [c + q for c, q in zip(ctxs, q_lens)]
    maxb = max(-(-s // ps) for s in sls)
    nb = len(sls) * maxb + 3
    perm = torch.randperm(nb, generator=g)[: len(sls) * maxb].to(torch.int32)
    bt = perm.reshape(len(sls), maxb)
    T = sum(q_lens)
    q = torch.randn(T, hq, d, generator=g).to(dtype)
    kv = torch.randn(nb, 2, ps, hkv, d, generator=g).to(dtype)
    qsl = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    sl = torch.tensor(sls, dtype=torch.int32)
    return q.to(DEV), kv.to(DEV), qsl.to(DEV), sl.to(DEV), bt.to(DEV)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d,ps,group", [(128, 16, 4), (64, 1, 1), (96, 32, 2), (128, 16, 8)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_workgroups_match_split_path(dtype, d, ps, group, causal):
    hkv = 2
    args = _prefix_case([300, 45, 130], [700, 0, 1500], hkv * group, hkv, d, ps, dtype, seed=d + ps + group)
    scale = 1 / math.sqrt(d)
    one = attend(*args, 300, 1, causal=causal, scale=scale)
    assert torch.equal(one, attend(*args, 300, 3, causal=causal, scale=scale))
    assert torch.equal(one, attend(*args, 300, 0, causal=causal, scale=scale))


@pytest.mark.parametrize("bits,frac", [(16, 8), (32, 16), (64, 32)])
def test_prefill_workgroups_formats_windows_alibi_softcap(bits, frac):
    dtype = torch.bfloat16
    args = _prefix_case([260, 140], [600, 50], 8, 2, 128, 16, dtype, seed=bits)
    slopes = torch.linspace(0.02, 0.5, 8, dtype=torch.float32, device=DEV)
    kw = dict(scale=1 / math.sqrt(128), bits=bits, frac=frac, alibi=slopes, softcap=20.0, window=333)
    one = attend(*args, 260, 1, **kw)
    assert torch.equal(one, attend(*args, 260, 4, **kw))
    tol = 5e-2 if bits == 16 else 1e-2
    assert close(one, oracle(*args, scale=kw["scale"], bits=bits, frac=frac, alibi=slopes, softcap=20.0,
                             window=333), tol)


@pytest.mark.parametrize("bits,frac", [(16, 8), (32, 16), (32, 32), (64, 32)])
@pytest.mark.parametrize("window", [0, 333])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_prefill_score_variants_match_split_path(bits, frac, window, sign):
    # the prefill workgroups' fast variant (no softcap / ALiBi, positive
    # scale, 2^f within the rounding constant's range: (16, 8) and (32, 16);
    # whole tiles unmasked, the row maximum taken before scaling) and their
    # general one ((32, 32), (64, 32), a negative scale) against the split
    # path, bit for bit, with NaN keys in one request
    dtype = torch.bfloat16
    q, kv, qsl, sl, bt = _prefix_case([260, 140], [600, 50], 8, 2, 128, 16, dtype, seed=bits + frac)
    kv[bt[0, 5].long(), 0, 3, 1, 7] = float("nan")  # key 83 of request 0, kv head 1
    kw = dict(scale=sign / math.sqrt(128), bits=bits, frac=frac, window=window)
    one = attend(q, kv, qsl, sl, bt, 260, 1, **kw)
    split = attend(q, kv, qsl, sl, bt, 260, 4, **kw)
    assert torch.equal(one.view(torch.int16), split.view(torch.int16))


@pytest.mark.parametrize("bits,frac", [(16, 8), (32, 16)])
def test_prefill_weighted_v_paths_match_split_path(bits, frac):
    # the fast prefill variant quantises a d block of weighted V by the
    # rounding constant when every partial is in range, else exactly: V dims
    # 32..47 of kv head 0 scaled by 2^12 push that block out of range (16-bit
    # sums saturate), the other blocks stay fast, and a NaN value sends its
    # block to the exact path; bits equal the split path's
    dtype = torch.bfloat16
    q, kv, qsl, sl, bt = _prefix_case([300, 180], [700, 90], 8, 2, 128, 16, dtype, seed=bits + 7)
    kv[:, 1, :, 0, 32:48] *= 4096
    kv[bt[1, 2].long(), 1, 5, 1, 70] = float("nan")  # V of key 37 of request 1, kv head 1
    kw = dict(scale=1 / math.sqrt(128), bits=bits, frac=frac)
    one = attend(q, kv, qsl, sl, bt, 300, 1, **kw)
    split = attend(q, kv, qsl, sl, bt, 300, 4, **kw)
    assert torch.equal(one.view(torch.int16), split.view(torch.int16))
    assert torch.isfinite(one[:300].float()).all()  # request 0 holds no NaN


def test_prefill_rows_equal_their_decode_step():
    # the last prompt token computed inside a 400-token prefill equals the
    # same token computed as a one-token decode over the cached prefix
    dtype = torch.bfloat16
    q, kv, qsl, sl, bt = _prefix_case([400], [900], 32, 8, 128, 16, dtype, seed=3)
    scale = 1 / math.sqrt(128)
    full = attend(q, kv, qsl, sl, bt, 400, 1, scale=scale)
    q1 = q[-1:].contiguous()
    dec = attend(q1, kv, torch.tensor([0, 1], dtype=torch.int32, device=DEV), sl, bt, 1, 0, scale=scale)
    assert torch.equal(full[-1:], dec)
    assert close(full, oracle(q, kv, qsl, sl, bt, scale=scale))


def test_mixed_batch_routes_each_request_and_keeps_bits():
    # decode steps, a short prompt (below the prefill-workgroup threshold)
    # and a long prompt in one launch: each request's output equals the
    # request run alone
    dtype = torch.bfloat16
    q_lens, ctxs = [1, 300, 1, 5, 1], [2000, 700, 517, 40, 3000]
    q, kv, qsl, sl, bt = _prefix_case(q_lens, ctxs, 32, 8, 128, 16, dtype, seed=21)
    scale = 1 / math.sqrt(128)
    both = attend(q, kv, qsl, sl, bt, max(q_lens), 0, scale=scale)
    starts = [0] + list(np.cumsum(q_lens))
    for i, ql in enumerate(q_lens):
        qi = q[starts[i]:starts[i] + ql].contiguous()
        alone = attend(qi, kv, torch.tensor([0, ql], dtype=torch.int32, device=DEV), sl[i:i + 1].contiguous(),
                       bt[i:i + 1].contiguous(), ql, 0, scale=scale)
        assert torch.equal(both[starts[i]:starts[i] + ql], alone), i


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_strided_query_and_output_views(dtype):
    # q as the leading columns of a fused q/k/v projection output and o as
    # columns of a wider buffer (token strides above heads x head_dim, as
    # vLLM hands them over): the same bits as contiguous tensors on the
    # decode, short-prompt and prefill-workgroup paths, split and unsplit,
    # and nothing written outside the view
    q_lens, ctxs = [1, 300, 1, 5, 1], [2000, 700, 517, 40, 3000]
    hq, hkv, d = 8, 2, 128
    q, kv, qsl, sl, bt = _prefix_case(q_lens, ctxs, hq, hkv, d, 16, dtype, seed=33)
    T = q.shape[0]
    qkv = torch.full((T, (hq + 2 * hkv) * d), float("nan"), dtype=dtype, device=DEV)
    qkv[:, :hq * d] = q.reshape(T, hq * d)
    qv = qkv[:, :hq * d].view(T, hq, d)
    assert qv.stride() == ((hq + 2 * hkv) * d, d, 1)
    scale = 1 / math.sqrt(d)
    for splits in (0, 1):
        want = attend(q, kv, qsl, sl, bt, max(q_lens), splits, scale=scale)
        buf = torch.full((T, hq * d + 64), 7.0, dtype=dtype, device=DEV)
        ov = buf[:, 32:32 + hq * d].view(T, hq, d)
        torch.ops.fxpr.unified_attention_fxp(qv, kv, ov, qsl, sl, bt, max(q_lens), None, True, scale, 32, 16,
                                             0.0, 0, splits)
        assert torch.equal(ov, want), splits
        assert torch.all(buf[:, :32] == 7.0) and torch.all(buf[:, 32 + hq * d:] == 7.0)


def test_long_context_decode_split_invariance_and_reference():
    # contexts of 131072 and 70001 keys (256 and 137 chunks of 512) beside a
    # short one: unsplit, auto, 7 and 64 splits and a request of 100 give the
    # same bits; each row is within the tolerance of a float64 softmax over
    # all its keys (the reference's one maximum per row), with 131072 keys in
    # the denominator's 32-bit fixed-point sum
    hq, hkv, d, ps = 32, 8, 128, 16
    lens = [131072, 70001, 600]
    maxb = max(lens) // ps
    pool = sum(-(-L // ps) for L in lens) + 5
    g = torch.Generator("cpu").manual_seed(8)
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    bt = torch.zeros(len(lens), maxb, dtype=torch.int32)
    at = 0
    for r, L in enumerate(lens):
        n = -(-L // ps)
        bt[r, :n] = perm[at:at + n]
        at += n
    gd = torch.Generator(DEV).manual_seed(9)
    kv = torch.randn(pool, 2, ps, hkv, d, generator=gd, device=DEV, dtype=torch.bfloat16)
    q = (torch.randn(len(lens), hq, d, generator=g) * 2.0).to(torch.bfloat16).to(DEV)
    qsl = torch.arange(len(lens) + 1, dtype=torch.int32, device=DEV)
    sl, btd = torch.tensor(lens, dtype=torch.int32, device=DEV), bt.to(DEV)
    scale = 1 / math.sqrt(d)
    ref = attend(q, kv, qsl, sl, btd, 1, 1, scale=scale)
    for s in (0, 7, 64, 100):
        assert torch.equal(attend(q, kv, qsl, sl, btd, 1, s, scale=scale), ref), s
    for r, L in enumerate(lens):
        n = -(-L // ps)
        pages = kv[bt[r, :n].long().to(DEV)]                     # [n, 2, ps, hkv, d]
        k = pages[:, 0].reshape(n * ps, hkv, d)[:L].double()
        v = pages[:, 1].reshape(n * ps, hkv, d)[:L].double()
        qh = q[r].double().view(hkv, hq // hkv, d)
        s_ = torch.matmul(qh, k.permute(1, 2, 0).contiguous()) * scale   # [hkv, group, L]
        p = torch.softmax(s_, dim=-1)
        want = torch.matmul(p, v.permute(1, 0, 2).contiguous()).reshape(hq, d)
        err = (ref[r].double() - want).abs()
        tol = 1e-2 * want.abs() + 1e-2 * want.pow(2).mean().sqrt()
        assert torch.all(err <= tol), (r, float((err - tol).max()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_prompt_prefill_reference(dtype):
    # a 4096-token prompt over a 1000-key cached prefix (causal, GQA 4):
    # unsplit and auto splits give the same bits, and sampled rows (chunk
    # and row-tile edges, the last row) are within the tolerance of a
    # float64 softmax over their keys
    hq, hkv, d, ps, ql, ctx = 32, 8, 128, 16, 4096, 1000
    q, kv, qsl, sl, bt = _prefix_case([ql], [ctx], hq, hkv, d, ps, dtype, seed=12)
    scale = 1 / math.sqrt(d)
    out = attend(q, kv, qsl, sl, bt, ql, 1, scale=scale)
    assert torch.equal(out, attend(q, kv, qsl, sl, bt, ql, 0, scale=scale))
    L = ctx + ql
    n = -(-L // ps)
    pages = kv[bt[0, :n].long()]
    k = pages[:, 0].reshape(n * ps, hkv, d)[:L].double().permute(1, 2, 0).contiguous()  # [hkv, d, L]
    v = pages[:, 1].reshape(n * ps, hkv, d)[:L].double().permute(1, 0, 2).contiguous()  # [hkv, L, d]
    g = torch.Generator("cpu").manual_seed(13)
    rows = sorted({0, 1, 63, 64, 511, 512, 2047, ql - 1} | set(torch.randint(0, ql, (16,), generator=g).tolist()))
    for i in rows:
        keys = ctx + i + 1
        qh = q[i].double().view(hkv, hq // hkv, d)
        p = torch.softmax(torch.matmul(qh, k[:, :, :keys]) * scale, dim=-1)
        want = torch.matmul(p, v[:, :keys]).reshape(hq, d)
        err = (out[i].double() - want).abs()
        tol = 1e-2 * want.abs() + 1e-2 * want.pow(2).mean().sqrt()
        assert torch.all(err <= tol), (i, float((err - tol).max()))


@pytest.mark.parametrize("ps", [16, 32, 64, 128, 256])
def test_page_sizes_decode_and_prefill(ps):
    # pages of 16 to 256 keys (the DMA kernels take a wave's 16 key rows from
    # one page): decode steps and a prompt in one launch, split and unsplit
    # bits equal, against the oracle
    q_lens, ctxs = [1, 1, 200, 1], [3000, 777, 300, 64]
    q, kv, qsl, sl, bt = _prefix_case(q_lens, ctxs, 16, 4, 128, ps, torch.bfloat16, seed=ps)
    scale = 1 / math.sqrt(128)
    one = attend(q, kv, qsl, sl, bt, max(q_lens), 1, scale=scale)
    for s in (0, 3):
        assert torch.equal(attend(q, kv, qsl, sl, bt, max(q_lens), s, scale=scale), one), s
    assert close(one, oracle(q, kv, qsl, sl, bt, scale=scale))
