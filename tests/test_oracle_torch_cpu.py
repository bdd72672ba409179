"""Pin oracle/torch_cpu.py (the PyTorch CPU emulation the benchmark times)
bit for bit against the numpy oracle it restates (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemm as G
from oracle import numerics as N
from oracle import rows as R
from oracle import torch_cpu as TC


def _t(a):
    a = np.asarray(a)
    return torch.from_numpy(a.astype(np.int32) if a.dtype == np.uint16 else a.copy())


def _same(a, b):
    a = a.numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    b = np.asarray(b)
    if b.dtype == np.uint16:
        return np.array_equal(a.astype(np.uint16), b)
    if np.issubdtype(b.dtype, np.floating):
        return np.array_equal(a.view(np.uint8), b.view(np.uint8)) or bool(
            np.all((a == b) | (np.isnan(a) & np.isnan(b))))
    return np.array_equal(a, b)


@pytest.mark.parametrize("b,f", [(32, 16), (64, 32), (16, 8), (64, 16)])
def test_casts(b, f):
    rng = np.random.default_rng(b + f)
    x = (rng.standard_normal(20000) * np.logspace(-8, 12, 20000)).astype(np.float32)
    x[:6] = [np.nan, np.inf, -np.inf, 0.5, -2.5, 3.5]
    q = TC.float_to_fixed(torch.from_numpy(x), b, f)
    assert np.array_equal(q.numpy(), N.float_to_fixed(x, b, f).astype(np.int64))
    qq = q.reshape(100, 200)
    if b < 64:
        assert np.array_equal(TC.fixed_row_sum(qq, b).numpy(), N.fixed_row_sum(qq.numpy().astype(N.INT_DTYPE_BY_BITS[b]), b))


@pytest.mark.parametrize("io", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("bits,frac", [(32, 16), (64, 16), (16, 8)])
def test_gemm(io, bits, frac):
    rng = np.random.default_rng(3)
    a = N.store(rng.standard_normal((37, 300)).astype(np.float32), io)
    b = N.store((rng.standard_normal((300, 65)) * 0.3).astype(np.float32), io)
    bias = N.store(rng.standard_normal(65).astype(np.float32), io)
    want = G.gemm(a, b, bias, io, bits, frac)
    assert _same(TC.gemm(_t(a), _t(b), _t(bias), io, bits, frac), want)


@pytest.mark.parametrize("io", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("residual", [False, True])
def test_rms_norm(io, residual):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((9, 1000)) * np.array([[1e-3], [1], [3], [20], [100], [1e4], [0], [1], [2]])).astype(np.float32)
    x[7, 5] = np.inf
    x[8, 9] = np.nan
    r = (rng.standard_normal((9, 1000)) * 2).astype(np.float32)
    w = (rng.standard_normal(1000) * 0.1 + 1).astype(np.float32)
    xs, rs, ws = N.store(x, io), N.store(r, io), N.store(w, io)
    y, nr = R.rms_norm(xs, ws, 1e-6, io, residual=rs if residual else None)
    ty, tnr = TC.rms_norm(_t(xs), _t(ws), 1e-6, io, residual=_t(rs) if residual else None)
    assert _same(ty, y)
    if residual:
        assert _same(tnr, nr)


@pytest.mark.parametrize("bits,frac", [(32, 16), (64, 32), (16, 8)])
@pytest.mark.parametrize("io_out", ["bf16", "f32"])
def test_log_softmax(bits, frac, io_out):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 5000)) * 4
    x[0] = 0.0
    x[1, ::7] = 30.0
    x[2, 3] = np.nan
    x[3] = -np.inf
    xs = N.store(x.astype(np.float32), "bf16")
    want = R.log_softmax(xs, "bf16", io_out, bits, frac)
    assert _same(TC.log_softmax(_t(xs), "bf16", io_out, bits, frac), want)


@pytest.mark.parametrize("io,b,f", [("bf16", 32, 16), ("f16", 64, 32), ("bf16", 16, 8)])
def test_decode_attention(io, b, f):
    # decode rows of several 512-key chunks (distinct chunk maxima), ragged
    # lengths and a shuffled page table, against the numpy oracle's chunked
    # algorithm
    from oracle import attention as OA

    rng = np.random.default_rng(7)
    R, Hq, Hkv, D, ps = 5, 8, 2, 64, 16
    sl = np.array([1, 70, 600, 1500, 2049], np.int32)
    nbk = [-(-int(L) // ps) for L in sl]
    NB = sum(nbk) + 4
    perm = rng.permutation(NB)
    bt = np.zeros((R, max(nbk)), np.int32)
    off = 0
    for i, n in enumerate(nbk):
        bt[i, :n] = perm[off:off + n]
        off += n
    kv = rng.standard_normal((NB, 2, ps, Hkv, D)).astype(np.float32) * 2.0
    q = rng.standard_normal((R, Hq, D)).astype(np.float32)
    kvs, qs = N.store(kv, io), N.store(q, io)
    want = OA.unified_attention(qs, kvs, np.arange(R + 1, dtype=np.int32), sl, bt, io, softmax_scale=D ** -0.5,
                                int_bits=b, frac_bits=f, chunk_keys=OA.CHUNK_KEYS)
    got = TC.decode_attention(_t(qs), _t(kvs), torch.from_numpy(sl), torch.from_numpy(bt), io, D ** -0.5, b, f)
    assert _same(got, want)
