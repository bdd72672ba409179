"""fxpr_unified_attention_noalloc (the entry point that allocates nothing)
against fxpr_unified_attention, through the C ABI.

Split launches put their partials in the library's static device array
instead of a caller workspace; the results must be the same bits. Two calls
in a row, the second with a smaller input (the array keeps the first call's
contents), int32 and int64 accumulators, and a launch whose partials exceed
the array, which must be rejected before anything runs.
"""

from __future__ import annotations

import pytest
import torch

import fxpr_vllm  # noqa: F401
from fxpr_vllm import _hip
from fxpr_vllm._kernels import attention as KA

pytestmark = pytest.mark.gpu
DEV = "cuda"
STATIC_BYTES = 64 << 20   # FXPR_STATIC_SCRATCH_BYTES in include/fxpr.h


def _decode(batch, ctx_hi, seed, hq=32, hkv=8, d=128, ps=16, q_len=1):
    g = torch.Generator("cpu").manual_seed(seed)
    sl = torch.randint(ctx_hi // 2, ctx_hi + 1, (batch,), generator=g, dtype=torch.int32)
    maxb = -(-int(sl.max()) // ps)
    nb = batch * maxb + 3
    bt = torch.randperm(nb, generator=g)[: batch * maxb].to(torch.int32).reshape(batch, maxb)
    q = torch.randn(batch * q_len, hq, d, generator=g).to(torch.bfloat16)
    kv = torch.randn(nb, 2, ps, hkv, d, generator=g).to(torch.bfloat16)
    qsl = torch.arange(0, batch * q_len + 1, q_len, dtype=torch.int32)
    return [t.to(DEV) for t in (q, kv, qsl, sl, bt)], q_len


def _run(args, q_len, splits, bits, static):
    q, kv, qsl, sl, bt = args
    o = torch.full_like(q, 7.0)
    KA.unified_attention_fxp_run(q, kv, o, qsl, sl, bt, q_len, None, True, None, bits, 16 if bits < 64 else 32,
                                 0.0, 0, splits, static_scratch=static)
    return o


def _need(args, q_len, splits, bits):
    q, kv, qsl, sl, bt = args
    return _hip.load().fxpr_attention_workspace_bytes(sl.shape[0], q.shape[0], q.shape[1], kv.shape[3], q.shape[2],
                                                      bits, splits, q_len, bt.shape[1], kv.shape[2])


@pytest.mark.parametrize("bits", [32, 64])
def test_noalloc_matches_workspace_entry_point_twice(bits):
    big, ql = _decode(64, 8192, seed=bits)            # the bench's decode shape, 16 splits
    small, ql2 = _decode(8, 1500, seed=bits + 1)     # then a smaller launch over the same array
    assert 0 < _need(big, ql, 16, bits) <= STATIC_BYTES
    assert 0 < _need(small, ql2, 4, bits) < _need(big, ql, 16, bits)
    for args, q_len, splits in ((big, ql, 16), (small, ql2, 4), (small, ql2, 0), (big, ql, 1)):
        want = _run(args, q_len, splits, bits, static=False)
        got = _run(args, q_len, splits, bits, static=True)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (splits, bits)


def test_noalloc_rejects_partials_beyond_the_array():
    args, q_len = _decode(4, 8000, seed=9, q_len=128)   # 512 query rows x 32 heads x 11 chunks x 128
    need = _need(args, q_len, 4, 32)
    assert need > STATIC_BYTES
    q = args[0]
    o = torch.full_like(q, 7.0)
    with pytest.raises(RuntimeError, match="workspace"):
        KA.unified_attention_fxp_run(q, *args[1:2], o, *args[2:], q_len, None, True, None, 32, 16, 0.0, 0, 4,
                                     static_scratch=True)
    torch.cuda.synchronize()
    assert torch.all(o == 7.0)   # nothing ran
    # the same launch with a caller workspace still works, and an unsplit
    # launch needs no scratch at all
    assert torch.equal(_run(args, q_len, 1, 32, static=True).view(torch.int16),
                       _run(args, q_len, 4, 32, static=False).view(torch.int16))
