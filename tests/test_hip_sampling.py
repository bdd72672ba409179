"""GPU parity: the greedy sampler (sample_greedy_fxp, DeterministicSampler).

Token ids and top-k ids equal the oracle's order exactly, log-probabilities
equal the oracle's and log_softmax_fxp's fp32 outputs bit for bit, at full
vocabulary and on tie-heavy, NaN, infinite and ragged rows; tokens equal
torch.argmax on finite rows; rows do not depend on the batch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import fxpr_vllm  # noqa: F401
from fxpr_vllm._kernels import sampling as KS
from fxpr_vllm.sampling import DeterministicSampler
from oracle import sampling as S
from tests._util import IO_NAME, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _logits(rows, vocab, seed, dtype=torch.bfloat16, ties=False):
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(rows, vocab, generator=g) * 4.0
    if ties:
        x = torch.round(x)
    return x.to(dtype)


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise equal fp32, any NaN matching any NaN (the host's default NaN
    carries the sign bit, the GPU's does not)."""
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) |
                                              (np.isnan(a) & np.isnan(b))))


def _check(x, k, b, f):
    got = KS.sample_greedy_fxp_run(x.to(DEV), k, b, f)
    ids, lp, top, top_lp = S.sample_greedy(to_np(x), IO_NAME[x.dtype], k, b, f)
    assert np.array_equal(got[0].cpu().numpy(), ids)
    assert _same_bits(got[1].cpu().numpy(), lp)
    assert np.array_equal(got[2].cpu().numpy(), top)
    assert _same_bits(got[3].cpu().numpy(), top_lp)
    return got


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("k", [0, 1, 20, 64])
def test_full_vocab_bit_exact(dtype, k):
    _check(_logits(8, 128_256, seed=k, dtype=dtype), k, 32, 16)


@pytest.mark.parametrize("b,f", [(32, 16), (64, 32), (16, 8), (64, 63)])
@pytest.mark.parametrize("shape", [(3, 1), (5, 7), (4, 1001), (2, 300_001)])
def test_formats_and_ragged_rows(b, f, shape):
    _check(_logits(*shape, seed=sum(shape), ties=True), min(5, shape[1]), b, f)


def test_special_rows():
    V = 4096
    x = torch.round(torch.randn(6, V, generator=torch.Generator("cpu").manual_seed(3)) * 2)
    x[1, 100] = float("nan")
    x[1, 3000] = float("nan")
    x[2] = 0.0
    x[2, ::2] = -0.0
    x[3, 5] = float("inf")
    x[3, 6] = float("inf")
    x[4] = -float("inf")
    x[5, :] = 7.0
    for dtype in (torch.float32, torch.bfloat16):
        ids = _check(x.to(dtype), 10, 32, 16)[0].cpu()
        assert ids.tolist()[1:] == [100, 0, 5, 0, 0]


def test_top_keys_held_by_few_threads():
    # The kernel keeps each thread's two largest keys and rescans a thread's
    # elements when it supplies a third winner. Rows whose top 64 lie in a
    # few threads' elements: a flat row (keys ordered by index: the first 64
    # elements), the top 64 values in one thread's chunks of 8 (thread 3 of
    # 512, chunks 3 + 512 i) in descending order, the same interleaved over
    # two threads with ties, and at the row's end.
    V = 128_256
    x = torch.round(torch.randn(4, V, generator=torch.Generator("cpu").manual_seed(9)) * 2)
    x[0] = 7.0
    pos = torch.tensor([8 * (3 + 512 * i) + j for i in range(8) for j in range(8)])
    x[1, pos] = 200.0 - torch.arange(64, dtype=torch.float32)
    pos2 = torch.tensor([8 * (t + 512 * i) + j for i in range(4) for t in (3, 4) for j in range(8)])
    x[2, pos2] = 150.0 - (torch.arange(64) // 3).to(torch.float32)
    x[3, V - 64:] = 100.0
    for dtype in (torch.bfloat16, torch.float32):
        ids = _check(x.to(dtype), 64, 32, 16)[2].cpu()
        assert ids[0].tolist() == list(range(64))
        assert ids[1].tolist() == pos.tolist()
        assert ids[3].tolist() == list(range(V - 64, V))


def _sample_both_paths(x, k, b, f):
    """The C entry point without a workspace (one workgroup per row) and with
    one (rows of at most 128 spread over several workgroups)."""
    from fxpr_vllm import _hip
    rows, vocab = x.shape
    outs = []
    for use_ws in (False, True):
        ids = torch.full((rows,), -1, dtype=torch.int64, device=DEV)
        lp = torch.full((rows,), 7.0, dtype=torch.float32, device=DEV)
        top = torch.full((rows, k), -1, dtype=torch.int64, device=DEV)
        top_lp = torch.full((rows, k), 7.0, dtype=torch.float32, device=DEV)
        ws_bytes = _hip.load().fxpr_sample_greedy_workspace_bytes(rows, k) if use_ws else 0
        ws = torch.full((max(ws_bytes, 1),), 0xA5, dtype=torch.uint8, device=DEV)  # stale contents
        _hip.call("fxpr_sample_greedy", x.data_ptr(), _hip.DTYPE_CODE[x.dtype], rows, vocab, k, b, f,
                  ids.data_ptr(), lp.data_ptr(), top.data_ptr() if k else None, top_lp.data_ptr() if k else None,
                  ws.data_ptr() if use_ws else None, ws_bytes, _hip.stream_ptr(x.device))
        outs.append((ids.cpu(), lp.cpu(), top.cpu(), top_lp.cpu()))
    return outs


def _paths_equal(one, multi):
    # ids exactly; log-probabilities bit for bit, any NaN matching any NaN (a
    # NaN row's payload may come from different operands on the two paths)
    assert torch.equal(one[0], multi[0]) and torch.equal(one[2], multi[2])
    assert _same_bits(one[1].numpy(), multi[1].numpy()) and _same_bits(one[3].numpy(), multi[3].numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,vocab", [(1, 128_256), (32, 128_256), (128, 32_000), (3, 300_001), (5, 8192)])
@pytest.mark.parametrize("k", [0, 5, 64])
def test_multi_workgroup_rows_equal_one_workgroup(dtype, rows, vocab, k):
    # several workgroups per row (span maxima and top keys, span sums against
    # the row maximum, a per-row merge) give the one-workgroup kernel's bits;
    # 300001 columns take element loads
    x = _logits(rows, vocab, seed=rows + vocab + k, dtype=dtype, ties=(k == 64))
    if rows >= 3:
        x[0] = 2.0                      # flat: the top 64 all in the first span
        x[1, vocab // 3] = float("nan")
        x[2, -5:] = float("inf")
    one, multi = _sample_both_paths(x.to(DEV), k, 32, 16)
    _paths_equal(one, multi)
    if rows == 1 or (rows == 32 and k == 5):  # and the oracle, for a few
        ids, lp, top, top_lp = S.sample_greedy(to_np(x), IO_NAME[x.dtype], k, 32, 16)
        assert np.array_equal(multi[0].numpy(), ids) and np.array_equal(multi[2].numpy(), top)
        assert _same_bits(multi[1].numpy(), lp) and _same_bits(multi[3].numpy(), top_lp)


@pytest.mark.parametrize("b,f", [(64, 32), (16, 8), (64, 63)])
def test_multi_workgroup_formats(b, f):
    # 64-bit (and 128-bit, Q63) exact sums and 16-bit terms across the spans
    x = _logits(16, 128_256, seed=b + f, ties=True)
    one, multi = _sample_both_paths(x.to(DEV), 10, b, f)
    _paths_equal(one, multi)


def test_logprobs_equal_log_softmax_and_tokens_equal_argmax():
    x = _logits(32, 128_256, seed=11).to(DEV)
    ids, lp, top, top_lp = torch.ops.fxpr.sample_greedy_fxp(x, 20, 32, 16)
    full = torch.ops.fxpr.log_softmax_fxp(x, 32, 16, torch.float32)
    assert torch.equal(ids, torch.argmax(x, dim=-1))
    assert torch.equal(lp.view(torch.int32), full.gather(1, ids[:, None])[:, 0].view(torch.int32))
    assert torch.equal(top_lp.view(torch.int32), full.gather(1, top).view(torch.int32))
    assert torch.all(top_lp[:, :-1] >= top_lp[:, 1:])


def test_batch_invariance_and_module():
    x = _logits(64, 32_000, seed=5).to(DEV)
    full = torch.ops.fxpr.sample_greedy_fxp(x, 8, 32, 16)
    for r in (0, 17, 63):
        one = torch.ops.fxpr.sample_greedy_fxp(x[r:r + 1].clone(), 8, 32, 16)
        for a, b in zip(one, full):
            assert torch.equal(a[0], b[r])
    out = DeterministicSampler()(x.view(4, 16, 32_000), num_logprobs=3)
    assert out.token_ids.shape == (4, 16) and out.topk_logprobs.shape == (4, 16, 3)
    assert torch.equal(out.token_ids.reshape(-1), full[0])
    assert torch.equal(out.topk_token_ids.reshape(64, 3), full[2][:, :3])
    lps = DeterministicSampler.compute_logprobs(x)
    assert torch.equal(lps.gather(1, full[0][:, None])[:, 0], full[1])


def test_errors():
    x = _logits(2, 100, seed=0).to(DEV)
    with pytest.raises(ValueError):
        torch.ops.fxpr.sample_greedy_fxp(x, 65, 32, 16)
    with pytest.raises(ValueError):
        torch.ops.fxpr.sample_greedy_fxp(x[:, :3], 4, 32, 16)
    with pytest.raises(ValueError):
        torch.ops.fxpr.sample_greedy_fxp(x, 2, 32, 12)
    with pytest.raises(TypeError):
        torch.ops.fxpr.sample_greedy_fxp(x.double(), 2, 32, 16)
    e = torch.ops.fxpr.sample_greedy_fxp(x[:0], 2, 32, 16)
    assert e[0].shape == (0,) and e[2].shape == (0, 2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("vocab_off", [-8, 0, 8])
def test_multi_workgroup_threshold(dtype, vocab_off):
    # rows split into spans only while every span keeps 256 threads' vectors:
    # at 512 vectors a row takes two spans, one vector less keeps one
    # workgroup; both sides of the threshold give the one-workgroup bits
    vec = 16 // torch.tensor([], dtype=dtype).element_size()
    vocab = 512 * vec + vocab_off
    x = _logits(6, vocab, seed=vocab, dtype=dtype, ties=True)
    x[2, -1] = float("inf")
    for k in (0, 7):
        one, multi = _sample_both_paths(x.to(DEV), k, 32, 16)
        _paths_equal(one, multi)
