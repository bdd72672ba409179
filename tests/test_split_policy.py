"""GPU-free decision tables of the split policies (host code of the C ABI).

The reference pins its GEMM split decision in a CPU test
(fxpr_vllm/_tests/test_gemm_warmup.py:16-62: cached choice, forced override,
clamps); its attention policy is closed-form (_pick_num_splits,
fxpr_vllm/_triton/attention.py:664-689). This build's policies are its own
static tables, in C (fxpr_attention_splits, fxpr_gemm_splits); these tests
pin them case by case. That a split count never changes the bits is the GPU
tests' part (tests/test_hip_attention.py, tests/test_hip_gemm.py).
"""

from __future__ import annotations

import pytest

from fxpr_vllm import _hip


@pytest.fixture(scope="module")
def lib():
    return _hip.load()


def attn_splits(lib, requests, kv_heads, group, max_q, keys, page=16, requested=0):
    return lib.fxpr_attention_splits(requests, kv_heads, group, max_q, -(-keys // page), page, requested)


def test_attention_explicit_request_wins(lib):
    # decode rows of 8192 keys hold 16 chunks of 512 keys
    for r in (1, 2, 3, 4, 8, 16):
        assert attn_splits(lib, 64, 8, 4, 1, 8192, requested=r) == r
    # an explicit request splits even where the automatic policy would not
    assert attn_splits(lib, 4, 8, 4, 1, 1024, requested=2) == 2          # short context
    assert attn_splits(lib, 1024, 8, 4, 1, 8192, requested=4) == 4      # oversubscribed
    assert attn_splits(lib, 4, 8, 4, 2048, 2048, requested=3) == 3       # prefill


def test_attention_explicit_request_beyond_chunks(lib):
    # splits past the row's chunk count would hold no keys: the launch runs
    # one per chunk (more than the automatic cap of 64 when rows are long)
    assert attn_splits(lib, 64, 8, 4, 1, 8192, requested=100) == 16
    assert attn_splits(lib, 2, 8, 4, 1, 65536, requested=100) == 100     # 128 chunks
    assert attn_splits(lib, 2, 8, 4, 1, 65536, requested=1000) == 128
    assert attn_splits(lib, 2, 8, 4, 1, 100, requested=5) == 1           # one chunk
    # the grid's z dimension bounds it
    assert attn_splits(lib, 1, 1, 1, 1, 512 * 70000, page=512, requested=70000) == 65535


def test_attention_auto_short_context(lib):
    # up to 32 key tiles of 64 (2048 keys): unsplit
    for keys in (1, 64, 512, 2048):
        assert attn_splits(lib, 4, 8, 4, 1, keys) == 1
    # 33 tiles: 5 chunks of 8 tiles, one split each
    assert attn_splits(lib, 4, 8, 4, 1, 2049) == 5


def test_attention_auto_one_chunk_per_split(lib):
    assert attn_splits(lib, 64, 8, 4, 1, 8192) == 16      # the bench decode shape
    assert attn_splits(lib, 64, 8, 4, 1, 4096) == 8
    assert attn_splits(lib, 1, 8, 4, 1, 20000) == 40      # ragged: 313 tiles, 40 chunks
    assert attn_splits(lib, 1, 8, 4, 1, 65536) == 64      # capped at 64
    assert attn_splits(lib, 1, 8, 4, 1, 1 << 20) == 64


def test_attention_auto_oversubscribed(lib):
    # (request, kv head, 16-row query tile) workgroups above 8 x 256: unsplit
    assert attn_splits(lib, 256, 8, 4, 1, 8192) == 16     # 2048 workgroups: still splits
    assert attn_splits(lib, 257, 8, 4, 1, 8192) == 1      # 2056
    # GQA groups share a query tile: 4 rows per (query, kv head) at group 4
    assert attn_splits(lib, 64, 8, 4, 4, 8192) == 16      # 16 rows: one tile
    assert attn_splits(lib, 64, 8, 4, 5, 8192) == 16      # 20 rows: 2 tiles, 1024 workgroups
    assert attn_splits(lib, 64, 8, 4, 17, 8192) == 1      # 68 rows: 5 tiles, 2560 workgroups
    # prefill: 4 requests x 8 kv heads x 512 query tiles
    assert attn_splits(lib, 4, 8, 4, 2048, 8192) == 1


def test_attention_policy_is_static(lib):
    # the same arguments always give the same count (graph capture bakes it in)
    first = [attn_splits(lib, b, 8, 4, 1, 8192) for b in (1, 8, 64, 300)]
    assert first == [attn_splits(lib, b, 8, 4, 1, 8192) for b in (1, 8, 64, 300)]


BF16, F16, F32 = 1, 0, 2


def gemm_splits(lib, m, n, k, dt=BF16, requested=0, bits=32):
    return lib.fxpr_gemm_splits(m, n, k, dt, bits, requested)


def test_gemm_explicit_request_wins(lib):
    # forced counts (the reference's _SPLITK_FORCE): honoured, clamped to the
    # K-tiles (128 wide for 16-bit inputs, 64 for fp32)
    assert gemm_splits(lib, 32, 4096, 4096, requested=4) == 4
    assert gemm_splits(lib, 1, 4096, 4096, requested=2) == 2          # even on a stream shape
    assert gemm_splits(lib, 8192, 128256, 4096, requested=3) == 3     # and a large one
    assert gemm_splits(lib, 32, 4096, 4096, requested=100) == 32      # 32 K-tiles
    assert gemm_splits(lib, 32, 4096, 4096, F32, requested=100) == 64
    assert gemm_splits(lib, 32, 4096, 128, requested=4) == 1          # one K-tile: never split
    assert gemm_splits(lib, 32, 4096, 0, requested=4) == 1
    assert gemm_splits(lib, 32, 4096, 129, requested=4) == 2          # a partial second tile


def test_gemm_auto_decode_shapes_stream(lib):
    # 16-bit, M <= 16, N <= 8192: the streaming kernel, never split
    for m in (1, 8, 16):
        for n in (1024, 4096, 6144, 8192):
            for k in (4096, 14336):
                assert gemm_splits(lib, m, n, k) == 1
                assert gemm_splits(lib, m, n, k, F16) == 1


def test_gemm_auto_split_fills_the_gpu(lib):
    # elsewhere: 512 / (output tiles) splits, at most 16, when the tiles do
    # not reach 256 (16 x 256 tiles for M <= 16; from M = 17 to 64 64 x 256
    # with 16- / 32-bit sums and 128 x 128 with 64-bit ones; 128 x 128 from
    # M = 65)
    assert gemm_splits(lib, 16, 8193, 4096) == 15        # 33 tiles
    assert gemm_splits(lib, 1, 28672, 4096) == 4         # 112 tiles
    assert gemm_splits(lib, 1, 128256, 4096) == 1        # 501 tiles
    assert gemm_splits(lib, 32, 4096, 4096) == 16        # 16 tiles
    assert gemm_splits(lib, 32, 6144, 4096) == 16        # 24 tiles
    assert gemm_splits(lib, 32, 28672, 4096) == 4        # 112 tiles
    assert gemm_splits(lib, 64, 28672, 4096, bits=16) == 4
    assert gemm_splits(lib, 32, 28672, 4096, bits=64) == 2    # 224 tiles
    assert gemm_splits(lib, 32, 6144, 4096, bits=64) == 10    # 48 tiles
    assert gemm_splits(lib, 65, 28672, 4096) == 2        # 224 tiles
    assert gemm_splits(lib, 256, 4096, 4096) == 8        # 64 tiles
    assert gemm_splits(lib, 32, 128256, 4096) == 1       # 501 tiles
    assert gemm_splits(lib, 8192, 128256, 4096) == 1
    assert gemm_splits(lib, 32, 4096, 256) == 2          # capped at the 2 K-tiles
    # fp32 inputs keep the skinny tiles (16 / 32 / 64 x 256) and 64-wide K-tiles
    assert gemm_splits(lib, 1, 4096, 4096, F32) == 16
    assert gemm_splits(lib, 32, 14336, 4096, F32) == 9   # 56 tiles
    assert gemm_splits(lib, 8192, 14336, 4096, F32) == 1


def test_gemm_workspace_follows_the_split(lib):
    # integer partials [splits, M, N] (4 or 8 bytes), none when unsplit
    assert lib.fxpr_gemm_workspace_bytes(32, 4096, 4096, BF16, 32, 0) == 16 * 32 * 4096 * 4
    assert lib.fxpr_gemm_workspace_bytes(32, 4096, 4096, BF16, 64, 0) == 16 * 32 * 4096 * 8
    assert lib.fxpr_gemm_workspace_bytes(1, 4096, 4096, BF16, 32, 0) == 0
    assert lib.fxpr_gemm_workspace_bytes(1, 4096, 4096, BF16, 32, 3) == 3 * 4096 * 4
    assert lib.fxpr_gemm_workspace_bytes(8192, 128256, 4096, BF16, 32, 0) == 0
