"""End-to-end batch invariance: a random-init Llama-shaped decoder built from
the fxpr ops (tests/e2e_decoder.py) generates greedily under different
schedules - requests alone (batch 1), together (batch 8 and 32), and a
continuous-batching mix where prefills join running decodes. Every request's
tokens, sampled-token log-probabilities and top-k log-probabilities (and, for
the small model, whole fixed-point log-probability rows) must be
bit-identical across schedules at every step. This is BASELINE config 5's
property (Llama-3-8B shape, prompts of 2048 tokens, batch 1/8/32) on the
library's own harness, without vLLM.
"""

from __future__ import annotations

import pytest
import torch

from e2e_decoder import Config, Decoder, run, run_graph

pytestmark = pytest.mark.gpu


def _prompts(n, seed=0, vocab=1024, lo=3, hi=40):
    g = torch.Generator("cpu").manual_seed(seed)
    lens = torch.randint(lo, hi, (n,), generator=g).tolist()
    return [torch.randint(0, vocab, (L,), generator=g).tolist() for L in lens]


def _bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t


def _assert_same(a, b, what=""):
    assert a.tokens == b.tokens, f"{what}: tokens differ"
    assert len(a.logprobs) == len(b.logprobs)
    for s in range(len(a.logprobs)):
        assert torch.equal(_bits(a.logprobs[s]), _bits(b.logprobs[s])), f"{what} step {s}: log-prob"
        assert torch.equal(a.topk[s][0], b.topk[s][0]), f"{what} step {s}: top-k ids"
        assert torch.equal(_bits(a.topk[s][1]), _bits(b.topk[s][1])), f"{what} step {s}: top-k log-probs"
    for s, (x, y) in enumerate(zip(a.full, b.full)):
        assert torch.equal(_bits(x), _bits(y)), f"{what} step {s}: log-prob row"


def _alone(step, active):
    return [min(active, key=lambda r: r.rid)]


def _all(step, active):
    return active


def _staggered(step, active):
    # admit two new requests per step while earlier ones keep decoding
    return [r for r in active if r.rid < 2 * (step + 1)]


def test_batch_1_vs_8_vs_mixed():
    import fxpr_vllm  # noqa: F401

    model = Decoder(Config())
    prompts = _prompts(8)
    ref = run(model, prompts, 6, _alone)
    for name, sched in (("batch 8", _all), ("mixed", _staggered)):
        got = run(model, prompts, 6, sched)
        for rid in ref:
            _assert_same(ref[rid], got[rid], f"{name} request {rid}")
    # the model is not degenerate: requests do not all emit the same tokens
    assert len({tuple(r.tokens[len(r.prompt):]) for r in ref.values()}) > 1
    # the sampled token is the row's argmax and its log-prob is the row's value
    for r in ref.values():
        for s, row in enumerate(r.full):
            tok = r.tokens[len(r.prompt) + s]
            assert tok == int(torch.argmax(row)) and torch.equal(_bits(row[tok]), _bits(r.logprobs[s]))


def test_graph_decode_matches_eager():
    # the serving loop the bench times: decode steps replayed from one
    # captured graph, state advanced on the device, pages assigned up front
    import fxpr_vllm  # noqa: F401

    model = Decoder(Config())
    prompts = _prompts(8, seed=3)
    ref = run(model, prompts, 6, _all)
    got = run_graph(model, prompts, 6)
    for rid in ref:
        _assert_same(ref[rid], got[rid], f"graph request {rid}")


def test_batch_32_matches_batch_1_subset():
    import fxpr_vllm  # noqa: F401

    model = Decoder(Config())
    prompts = _prompts(32, seed=1)
    big = run(model, prompts, 3, _all)
    for rid in (0, 13, 31):
        _assert_same(big[rid], run(model, [prompts[rid]], 3, _all)[0], f"request {rid}")


# --- the Llama-3-8B shape --------------------------------

PROMPT_LEN, BATCH, MAX_NEW = 2048, 32, 128


@pytest.fixture(scope="module")
def llama3_8b():
    import fxpr_vllm  # noqa: F401

    pages = BATCH * -(-(PROMPT_LEN + MAX_NEW) // 16) + 8
    model = Decoder(Config.llama3_8b(pages), seed=0)
    prompts = _prompts(BATCH, seed=5, vocab=128_256, lo=PROMPT_LEN, hi=PROMPT_LEN + 1)
    yield model, prompts
    del model
    torch.cuda.empty_cache()


def test_llama3_8b_shape_batch_1_8_32(llama3_8b):
    # 32 random-token prompts of 2048, greedy 128 tokens with the top-5
    # log-probabilities: batch 32, its first 8 as batch 8, three requests
    # alone, four requests staggered so prefills join running decodes, and
    # batch 32 again with its decode steps replayed from a captured graph
    model, prompts = llama3_8b
    b32 = run(model, prompts, MAX_NEW, _all)
    b8 = run(model, prompts[:8], MAX_NEW, _all)
    for rid in range(8):
        _assert_same(b32[rid], b8[rid], f"batch 8 request {rid}")
    for rid in (0, 19, 31):
        _assert_same(b32[rid], run(model, [prompts[rid]], MAX_NEW, _all)[0], f"alone request {rid}")
    mixed = run(model, prompts[8:12], MAX_NEW, _staggered)
    for i in range(4):
        _assert_same(b32[8 + i], mixed[i], f"staggered request {8 + i}")
    # the bench's serving loop: decode replayed from a captured graph
    g32 = run_graph(model, prompts, MAX_NEW)
    for rid in range(BATCH):
        _assert_same(b32[rid], g32[rid], f"graph request {rid}")
    generated = {tuple(r.tokens[PROMPT_LEN:]) for r in b32.values()}
    assert len(generated) > 1
    assert all(len(r.tokens) == PROMPT_LEN + MAX_NEW for r in b32.values())
