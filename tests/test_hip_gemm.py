"""GPU parity: fixed-point GEMM (HIP/MFMA) vs the oracle and the reference's
own GEMM tests (fxpr_vllm/_tests/test_gemm.py), restated.

Bit-exact against the oracle where every K-tile dot is exact in fp32 (small
integer inputs); within 1e-2 relative on seeded
N(0,1) data; bitwise invariant to split count, B layout, tile configuration
(batch size), K-tile permutation and repetition.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import fxpr_vllm  # noqa: F401
from fxpr_vllm._kernels import gemm as KG
from oracle import gemm as G
from tests._util import IO_NAME, close_report, from_np, mismatch_report, nan_aware_equal, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _int_mats(M, K, N, seed, lo=-2, hi=2, dtype=torch.bfloat16):
    g = torch.Generator("cpu").manual_seed(seed)
    a = torch.randint(lo, hi + 1, (M, K), generator=g).to(dtype)
    b = torch.randint(lo, hi + 1, (K, N), generator=g).to(dtype)
    return a, b


def _run(a, b, bias=None, bits=32, frac=16, split_k=0, b_layout="kn"):
    """b_layout 'kn': B row-major [K,N]; 'nk': B is the transpose view of a
    row-major [N,K] weight (how the vLLM glue stores it)."""
    ad = a.to(DEV)
    bd = b.to(DEV) if b_layout == "kn" else b.t().contiguous().to(DEV).t()
    bias_d = None if bias is None else bias.to(DEV)
    return KG.gemm_fxp_run(ad, bd, bias_d, bits, frac, split_k=split_k).cpu()


def _oracle(a, b, bias, bits, frac):
    io = IO_NAME[a.dtype]
    return from_np(G.gemm(to_np(a), to_np(b), None if bias is None else to_np(bias), io, bits, frac), a.dtype)


SHAPES = [(1, 1, 1), (3, 33, 7), (17, 257, 300), (40, 72, 300), (64, 512, 1000), (130, 33, 130), (200, 4096, 256)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("bits,frac", [(32, 16), (64, 16), (16, 8), (64, 32)])
@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("b_layout", ["kn", "nk"])
def test_gemm_exact_small_integers(dtype, bits, frac, M, K, N, b_layout):
    a, b = _int_mats(M, K, N, seed=M * 7 + K, dtype=dtype)
    got = _run(a, b, bits=bits, frac=frac, b_layout=b_layout)
    want = _oracle(a, b, None, bits, frac)
    assert torch.equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,K,N", [(1, 4096, 2048), (32, 4096, 2048), (256, 4096, 1024), (130, 130, 33)])
def test_gemm_tolerance_vs_oracle(dtype, M, K, N):
    g = torch.Generator("cpu").manual_seed(M + N)
    a = torch.randn(M, K, generator=g).to(dtype)
    b = (torch.randn(K, N, generator=g) * 0.02).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    want = _oracle(a, b, bias, 32, 16)
    for layout in ("kn", "nk"):
        got = _run(a, b, bias, b_layout=layout)
        # per element within 1e-2 relative
        report = close_report(got, want)
        assert not report, report


@pytest.mark.parametrize("dtype", DTYPES)
def test_gemm_split_and_layout_invariance(dtype):
    # split counts that the reduce kernel takes in batches of 8 and 4 splits
    # and singly; M x N = 48 x 520 takes its 16-byte loads, 47 x 519 (not a
    # multiple of 4 elements) its element loads
    g = torch.Generator("cpu").manual_seed(5)
    a = torch.randn(48, 2048 + 40, generator=g).to(dtype)
    b = torch.randn(2048 + 40, 520, generator=g).to(dtype)
    bias = torch.randn(520, generator=g).to(dtype)
    for m, n in ((48, 520), (47, 519)):
        am, bn, biasn = a[:m], b[:, :n], bias[:n]
        ref = _run(am, bn, biasn, split_k=1)
        for s in (0, 2, 3, 4, 7, 13, 16, 64):
            for layout in ("kn", "nk"):
                got = _run(am, bn, biasn, split_k=s, b_layout=layout, bits=32)
                assert torch.equal(got, ref), (m, n, s, layout, mismatch_report(got, ref))
        ref64 = _run(am, bn, biasn, split_k=1, bits=64)
        for s in (5, 12):
            assert torch.equal(_run(am, bn, biasn, split_k=s, bits=64, b_layout="nk"), ref64), (m, n, s)


@pytest.mark.parametrize("dtype", DTYPES)
def test_gemm_batch_size_invariance(dtype):
    # fxpr_vllm/_tests/test_gemm.py:245-269, extended over the tile configs
    g = torch.Generator("cpu").manual_seed(2026)
    K, N = 4096, 384
    a_full = torch.randn(300, K, generator=g).to(dtype)
    b = torch.randn(K, N, generator=g).to(dtype)
    bd = b.t().contiguous().to(DEV).t()
    rows = [0, 3, 17, 64, 127, 299]
    refs = {m: KG.gemm_fxp_run(a_full[m:m + 1].to(DEV), bd, None, 32, 16).cpu()[0] for m in rows}
    for batch in (1, 4, 16, 20, 33, 64, 65, 128, 300):
        out = KG.gemm_fxp_run(a_full[:batch].to(DEV), bd, None, 32, 16).cpu()
        for m in rows:
            if m < batch:
                assert torch.equal(out[m], refs[m]), (batch, m)


@pytest.mark.parametrize("dtype", DTYPES)
def test_gemm_ktile_permutation_invariance(dtype):
    # fxpr_vllm/_tests/test_gemm.py:214-242
    g = torch.Generator("cpu").manual_seed(123)
    kt = KG._BLOCK_K_BY_DTYPE[dtype]
    a = torch.randn(4, kt * 4, generator=g).to(dtype)
    b = torch.randn(kt * 4, 4, generator=g).to(dtype)
    perm = torch.cat([torch.arange(t * kt, (t + 1) * kt) for t in (2, 0, 3, 1)])
    assert torch.equal(_run(a, b), _run(a[:, perm], b[perm]))


def test_gemm_deterministic_across_runs():
    g = torch.Generator("cpu").manual_seed(77)
    a = torch.randn(512, 4096, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(4096, 2048, generator=g).to(torch.bfloat16).to(DEV)
    r0 = KG.gemm_fxp_run(a, b, None, 32, 16)
    for _ in range(4):
        assert torch.equal(r0, KG.gemm_fxp_run(a, b, None, 32, 16))


# --- large-M kernel: rounding-constant quantisation and its exact fallback ---
# gemm_big_kernel (16-bit inputs, M > 16, K-contiguous B) quantises a wave's
# K-tile by the rounding constant 1.5 * 2^23 when every partial satisfies
# |P| < 2^22 / 2^f (32767 / 2^f for 16-bit accumulators), and exactly
# otherwise. Inputs below keep every K-tile dot exact in fp32, so the result
# must equal the oracle bit for bit on either path.

# 128 x 128 tiles. Unsplit launches with 64-bit sums (fewer than 512
# K-tiles, f <= 20) run the 32-bit schedule plus the 64-bit redo of marked
# tiles at every M > 16; split ones the 64-bit kernel.
_BIG_M = [256, 1024]


def _dyadic(shape, lo, hi, exp2, g, dtype):
    return (torch.randint(lo, hi + 1, shape, generator=g).double() * 2.0 ** exp2).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", _BIG_M)
@pytest.mark.parametrize("bits,frac", [(32, 16), (16, 8), (32, 8), (16, 12), (64, 16)])
@pytest.mark.parametrize("K", [384, 300])
def test_gemm_big_rounding_constant_ties(dtype, M, bits, frac, K):
    # products are multiples of 2^-(f+1): many partials lie exactly halfway
    # between two fixed-point steps (round half to even), all far inside the
    # fast range; K = 300 adds the peeled partial last K-tile
    g = torch.Generator("cpu").manual_seed(M + frac + K)
    u = (frac + 1) // 2
    a = _dyadic((M, K), -8, 8, -u, g, dtype)
    b = _dyadic((K, 256), -8, 8, -(frac + 1 - u), g, dtype)
    got = _run(a, b, bits=bits, frac=frac, b_layout="nk")
    want = _oracle(a, b, None, bits, frac)
    assert torch.equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [17, 32, 48, 64])
def test_gemm_big_64x256_tiles_exact(dtype, M):
    # M = 17 .. 64 with 16- / 32-bit sums: 64 x 256 tiles (N = 520: three
    # column tiles, the last ragged). Dyadic inputs keep every K-tile dot
    # exact, so the result equals the oracle bit for bit: ties of the
    # rounding-constant path (K = 300: the peeled partial last K-tile), K-tiles
    # beyond the fast range (exact path), non-finite partials, and split
    # launches equal to the unsplit one
    g = torch.Generator("cpu").manual_seed(300 + M)
    N = 520
    for K in (300, 640):
        for bits, frac in ((32, 16), (16, 8), (32, 8)):
            u = (frac + 1) // 2
            a = _dyadic((M, K), -8, 8, -u, g, dtype)
            b = _dyadic((K, N), -8, 8, -(frac + 1 - u), g, dtype)
            got = _run(a, b, bits=bits, frac=frac, b_layout="nk")
            want = _oracle(a, b, None, bits, frac)
            assert torch.equal(got, want), (K, bits, frac, mismatch_report(got, want))
            for s in (2, 3):
                assert torch.equal(_run(a, b, bits=bits, frac=frac, b_layout="nk", split_k=s), want), (K, bits, s)
    K = 512
    a = _dyadic((M, K), -2, 2, -6, g, dtype)
    b = _dyadic((K, N), -2, 2, 0, g, dtype)
    a[M // 2, 128:256] *= 256  # one row's second K-tile beyond the fast range
    a[3, 0:128] *= 256
    a[1, 10] = float("inf")
    a[M - 1, 300] = float("nan")
    b[17, 9] = float("nan")
    for bits in (32, 16):
        frac = 8 if bits == 16 else 16
        want = _oracle(a, b, None, bits, frac)
        for s in (1, 4):
            got = _run(a, b, bits=bits, frac=frac, b_layout="nk", split_k=s)
            assert torch.equal(got, want), (bits, s, mismatch_report(got, want))


@pytest.mark.parametrize("seed", range(4))
def test_gemm_big_64x256_tiles_random_shapes(seed):
    # seeded random shapes of the M = 17 .. 64 tiles: M, N, K (K 16-byte
    # aligned rows, so the large-M kernel takes them; a partial last K-tile
    # when K is not a multiple of 128), accumulator width, split count and
    # input type; dyadic inputs (every K-tile dot exact) equal the oracle bit
    # for bit
    rng = np.random.default_rng(1000 + seed)
    for _ in range(6):
        M = int(rng.integers(17, 65))
        N = int(rng.integers(1, 700))
        K = 8 * int(rng.integers(1, 80))
        bits, frac = [(32, 16), (16, 8), (32, 12)][int(rng.integers(0, 3))]
        dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
        split = [0, 1, 2, 3, 5][int(rng.integers(0, 5))]
        g = torch.Generator("cpu").manual_seed(int(rng.integers(0, 1 << 30)))
        u = (frac + 1) // 2
        a = _dyadic((M, K), -8, 8, -u, g, dtype)
        b = _dyadic((K, N), -8, 8, -(frac + 1 - u), g, dtype)
        got = _run(a, b, bits=bits, frac=frac, b_layout="nk", split_k=split)
        want = _oracle(a, b, None, bits, frac)
        assert torch.equal(got, want), (M, N, K, bits, frac, dtype, split, mismatch_report(got, want))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", _BIG_M)
def test_gemm_big_mixed_tile_paths(dtype, M):
    # some waves' K-tiles hold partials beyond the fast range (|P| up to 2048
    # against 64 at Q16): those tiles take the exact path, the wave's other
    # tiles and the other waves the rounding constant
    g = torch.Generator("cpu").manual_seed(11 + M)
    K, N = 512, 256
    a = _dyadic((M, K), -2, 2, -6, g, dtype)
    b = _dyadic((K, N), -2, 2, 0, g, dtype)
    a[64:128, 128:256] *= 256  # one wave row, second K-tile
    a[M - 64:M - 48, 384:512] *= 256  # 16 rows of one wave, last K-tile
    a[3, 0:128] *= 256  # a single row, first K-tile
    for bits in (32, 16, 64):
        frac = 8 if bits == 16 else 16
        got = _run(a, b, bits=bits, frac=frac, b_layout="nk")
        want = _oracle(a, b, None, bits, frac)
        assert torch.equal(got, want), (bits, mismatch_report(got, want))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", _BIG_M)
def test_gemm_big_nonfinite_partials(dtype, M):
    # NaN and infinite partials fail the range check (the exact path turns
    # NaN into 0 and saturates infinities); the rest of their waves' tiles
    # are unaffected
    g = torch.Generator("cpu").manual_seed(5 + M)
    K, N = 384, 256
    a = _dyadic((M, K), -2, 2, -4, g, dtype)
    b = _dyadic((K, N), -2, 2, 0, g, dtype)
    a[5, 10] = float("inf")
    a[70, 300] = float("-inf")
    a[130, 200] = float("nan")
    b[17, 9] = float("nan")
    if dtype == torch.bfloat16:
        a[200, 140] = 2.0 ** 100  # finite inputs whose products overflow fp32
        b[140, :] = b[140, :] * 2.0 ** 30
    for bits in (32, 64):
        got = _run(a, b, bits=bits, frac=16, b_layout="nk")
        want = _oracle(a, b, None, bits, 16)
        assert torch.equal(got, want), (bits, mismatch_report(got, want))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", _BIG_M)
def test_gemm_big_split_k_invariance(dtype, M):
    # the large-M kernel's split-K instantiation: each split's K-tiles (with a
    # partial last tile in the last split) through the same rounding-constant
    # path, partial sums in the workspace, then the reduce; every split count
    # gives the unsplit bits, which equal the oracle on exact dots
    g = torch.Generator("cpu").manual_seed(17 + M)
    K, N = 1000, 384
    a = _dyadic((M, K), -3, 3, -5, g, dtype)
    b = _dyadic((K, N), -3, 3, 0, g, dtype)
    a[M // 2:M // 2 + 16, 256:384] *= 512  # one K-tile of some rows on the exact path
    want = _oracle(a, b, None, 32, 16)
    for s in (1, 2, 3, 5, 8):  # 5: the last split has no K-tiles
        got = _run(a, b, bits=32, frac=16, split_k=s, b_layout="nk")
        assert torch.equal(got, want), (s, mismatch_report(got, want))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1024, 64, 32])
def test_gemm_int64_marked_tile_redo(dtype, M):
    # unsplit 64-bit sums at M > 16 and f <= 20: 32-bit sums, tiles with a
    # K-tile outside the rounding-constant range marked (NaN at the tile's
    # first element) and recomputed by the 64-bit kernel (M = 32 / 64: the
    # decode-sized rows, unsplit on request). Here some K-tiles' quantised
    # partials exceed 2^31 (a 32-bit sum would saturate) and a NaN bias
    # column marks tiles that are in range (a redundant recompute); every row
    # equals the same row of split launches of half the rows (the 64-bit
    # kernel throughout) bit for bit, NaN for NaN
    g = torch.Generator("cpu").manual_seed(77 + M)
    K, N = 1024, 384
    a = torch.randn(M, K, generator=g).to(dtype)
    b = (torch.randn(K, N, generator=g) * 0.05).to(dtype)
    r0 = M // 5
    # bf16: |P * 2^16| mostly beyond 2^31; f16 (max 65504): beyond the range check only
    a[r0:r0 + 10, 128:256] = (a[r0:r0 + 10, 128:256].float() * (1e5 if dtype == torch.bfloat16 else 1e4)).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    bias[128] = float("nan")
    full = _run(a, b, bias, bits=64, frac=16, b_layout="nk", split_k=1)
    assert torch.isnan(full[:, 128]).all() and not torch.isnan(full[:, :128]).any()
    half = M // 2
    for m0 in (0, half):
        part = _run(a[m0:m0 + half].contiguous(), b, bias, bits=64, frac=16, b_layout="nk", split_k=2)
        assert nan_aware_equal(part, full[m0:m0 + half]), (m0, mismatch_report(part, full[m0:m0 + half]))
    want = _oracle(a[r0 - 5:r0 + 15], b, bias, 64, 16)
    report = close_report(full[r0 - 5:r0 + 15], want)
    assert not report, report


def test_gemm_int64_redo_groups():
    # The 64-bit redo pass checks the marking launch's tiles 64 per
    # workgroup: 8 x 65 = 520 tiles here (nine groups, the last of 8 tiles),
    # marks in several groups and several per group (NaN bias columns in
    # column tiles 0, 31, 64; out-of-range K-tiles in one row tile), and
    # every tile must equal the 64-bit kernel's (split launches) bit for bit
    g = torch.Generator("cpu").manual_seed(1234)
    M, K, N = 1024, 512, 8320
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = (torch.randn(K, N, generator=g) * 0.05).to(torch.bfloat16)
    a[300:310, 0:128] = (a[300:310, 0:128].float() * 1e5).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    for col in (5, 31 * 128 + 7, 64 * 128 + 1):
        bias[col] = float("nan")
    full = _run(a, b, bias, bits=64, frac=16, b_layout="nk", split_k=1)
    ref = _run(a, b, bias, bits=64, frac=16, b_layout="nk", split_k=2)
    assert nan_aware_equal(full, ref), mismatch_report(full, ref)
    assert torch.isnan(full[:, 5]).all() and not torch.isnan(full[:, 6]).any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_gemm_decode_shape_kernel_matches_split_path(dtype, M):
    # 16-bit inputs, M <= 16, N <= 8192, K a multiple of 128, K-contiguous B
    # (the linear layout): the decode-shape kernel (each workgroup 16 columns
    # over all of K, its four waves on contiguous K-tile runs, the sums added
    # through LDS). An explicit split request takes the 16 x 256 tiles split
    # over K instead. Same bits, equal to the oracle on exact dots, with a
    # ragged N, a bias and each accumulator width; K-tile counts below, at and
    # not a multiple of the wave count; every row equals an M = 1 launch of it
    g = torch.Generator("cpu").manual_seed(31 + M)
    for K, N in ((128, 1000), (384, 16), (640, 4096), (4096, 8192)):
        a = _dyadic((M, K), -3, 3, -5, g, dtype)
        b = _dyadic((K, N), -3, 3, 0, g, dtype)
        bias = _dyadic((N,), -8, 8, -3, g, dtype)
        for bits, frac in ((32, 16), (64, 16), (16, 8)):
            got = _run(a, b, bias, bits=bits, frac=frac, b_layout="nk")
            split = _run(a, b, bias, bits=bits, frac=frac, b_layout="nk", split_k=2)
            assert torch.equal(got, split), (K, N, bits, mismatch_report(got, split))
            want = _oracle(a, b, bias, bits, frac)
            assert torch.equal(got, want), (K, N, bits, mismatch_report(got, want))
        row = _run(a[M - 1:].contiguous(), b, bias, b_layout="nk")
        assert torch.equal(row[0], _run(a, b, bias, b_layout="nk")[M - 1])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M", [1, 8, 32, 64, 256])
def test_gemm_row_strided_a(dtype, M):
    # A as a view of wider rows (row stride above K, as a column slice of a
    # fused projection's output is): rows 16-byte aligned (8 elements of
    # padding: the vector, DMA and decode-shape paths) and not (3: element
    # loads). Bits equal the contiguous A's and the oracle's on exact dots,
    # at every M kernel family (decode-shape, 64 x 256, 128 x 128 tiles)
    g = torch.Generator("cpu").manual_seed(900 + M)
    K, N = 1024, 640
    for pad in (8, 3):
        wide = _dyadic((M, K + pad), -3, 3, -5, g, dtype)
        b = _dyadic((K, N), -3, 3, 0, g, dtype)
        bias = _dyadic((N,), -8, 8, -3, g, dtype)
        ad = wide.to(DEV)[:, :K]
        assert ad.stride() == (K + pad, 1)
        bd = b.t().contiguous().to(DEV).t()
        bias_d = bias.to(DEV)
        for bits, frac in ((32, 16), (64, 16)):
            got = KG.gemm_fxp_run(ad, bd, bias_d, bits, frac).cpu()
            dense = KG.gemm_fxp_run(ad.contiguous(), bd, bias_d, bits, frac).cpu()
            assert torch.equal(got, dense), (pad, bits, mismatch_report(got, dense))
            want = _oracle(wide[:, :K].contiguous(), b, bias, bits, frac)
            assert torch.equal(got, want), (pad, bits, mismatch_report(got, want))


# --- restated reference tests (fxpr_vllm/_tests/test_gemm.py) ---------------

@pytest.mark.parametrize("M,N,K", [(4, 4, 16), (3, 7, 16), (1, 1, 32), (8, 16, 32)])
def test_reference_gemm_correctness(M, N, K):
    g = torch.Generator("cpu").manual_seed(42)
    a = torch.randn(M, K, generator=g).to(DEV)
    b = torch.randn(K, N, generator=g).to(DEV)
    got = torch.ops.fxpr.gemm_fxp(a, b, None, 32, 16)
    assert torch.allclose(got, a @ b, atol=5e-4, rtol=5e-4)


def test_reference_gemm_identity_zero_single():
    g = torch.Generator("cpu").manual_seed(0)
    a = torch.randn(4, 16, generator=g).to(DEV)
    assert torch.allclose(torch.ops.fxpr.gemm_fxp(a, torch.eye(16, device=DEV), None, 32, 16), a, atol=1e-4)
    z = torch.ops.fxpr.gemm_fxp(torch.ones(4, 16, device=DEV), torch.zeros(16, 4, device=DEV), None, 32, 16)
    assert torch.equal(z, torch.zeros(4, 4, device=DEV))
    a1 = torch.randn(1, 16, generator=g).to(DEV)
    b1 = torch.randn(16, 1, generator=g).to(DEV)
    assert torch.allclose(torch.ops.fxpr.gemm_fxp(a1, b1, None, 32, 16), a1 @ b1, atol=5e-4)


_TOL = {torch.float32: 5e-4, torch.float16: 1e-2, torch.bfloat16: 5e-2}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,N,K", [(8, 16, 32), (4, 4, 64), (130, 130, 33), (4, 4, 33)])
def test_reference_gemm_with_bias(dtype, M, N, K):
    g = torch.Generator("cpu").manual_seed(123)
    a = (torch.randn(M, K, generator=g) * 0.5).to(dtype).to(DEV)
    b = (torch.randn(K, N, generator=g) * 0.5).to(dtype).to(DEV)
    bias_f32 = torch.randn(N, generator=g).to(DEV)
    got = torch.ops.fxpr.gemm_fxp(a, b, bias_f32.to(dtype), 32, 16)
    assert got.dtype == dtype and got.shape == (M, N)
    ref = (a.float() @ b.float() + bias_f32).to(dtype)
    tol = _TOL[dtype]
    assert torch.allclose(got.float(), ref.float(), atol=tol, rtol=tol)


def test_reference_gemm_large_shape_and_int_bits():
    g = torch.Generator("cpu").manual_seed(5)
    a = (torch.randn(256, 256, generator=g) * 0.3).to(DEV)
    b = (torch.randn(256, 256, generator=g) * 0.3).to(DEV)
    bias = torch.randn(256, generator=g).to(DEV)
    assert torch.allclose(torch.ops.fxpr.gemm_fxp(a, b, bias, 32, 16), a @ b + bias, atol=1e-3, rtol=1e-3)
    for bits in (32, 64):
        a2 = (torch.randn(4, 16, generator=g) * 0.25).to(DEV)
        b2 = (torch.randn(16, 4, generator=g) * 0.25).to(DEV)
        assert torch.allclose(torch.ops.fxpr.gemm_fxp(a2, b2, None, bits, 16), a2 @ b2, atol=5e-2, rtol=5e-2)


def test_gemm_errors_and_empty():
    a = torch.ones(4, 8, device=DEV)
    with pytest.raises(ValueError):
        torch.ops.fxpr.gemm_fxp(a, torch.ones(8, 4, device=DEV), None, 24, 16)
    with pytest.raises(TypeError):
        torch.ops.fxpr.gemm_fxp(a, torch.ones(8, 4, device=DEV, dtype=torch.float16), None, 32, 16)
    e = torch.ops.fxpr.gemm_fxp(torch.ones(0, 8, device=DEV), torch.ones(8, 4, device=DEV), None, 32, 16)
    assert e.shape == (0, 4)
    z = torch.ops.fxpr.gemm_fxp(torch.ones(3, 0, device=DEV), torch.ones(0, 4, device=DEV), None, 32, 16)
    assert torch.equal(z, torch.zeros(3, 4, device=DEV))


def test_lm_head_full_vocab_properties():
    # config-3 shape at M=1 and M=32: full N=128256, K=4096. Batch invariance
    # across the skinny (M = 1, 16) and large-M (M = 32) tiles, split
    # invariance, and an oracle check on a column sample (the oracle at full
    # size would take minutes).
    g = torch.Generator("cpu").manual_seed(0)
    K, N = 4096, 128256
    a = torch.randn(32, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bd = w.to(DEV).t()
    c32 = KG.gemm_fxp_run(a.to(DEV), bd, None, 32, 16)
    c1 = KG.gemm_fxp_run(a[:1].to(DEV), bd, None, 32, 16)
    assert torch.equal(c1[0], c32[0])
    c16 = KG.gemm_fxp_run(a[:16].to(DEV), bd, None, 32, 16)
    assert torch.equal(c16, c32[:16])
    c32s = KG.gemm_fxp_run(a.to(DEV), bd, None, 32, 16, split_k=4)
    assert torch.equal(c32s, c32)
    cols = torch.randperm(N, generator=g)[:512]
    want = _oracle(a, w[cols].t().contiguous(), None, 32, 16)
    report = close_report(c32.cpu()[:, cols], want)
    assert not report, report


# --- the benchmark's own shapes (BASELINE config 3 and 3') -----------------
# K = 4096 is 32 K-tiles: the large-M kernels' LDS rings wrap many times.


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1024, 2048])
@pytest.mark.parametrize("bits,frac", [(32, 16), (64, 16), (64, 24)])
def test_gemm_k4096_steady_state_exact(dtype, M, bits, frac):
    # dyadic inputs whose tile dots are exact in fp32 (|P| up to 2^13 * 2^-7
    # against the fast range 2^6 at Q16: a mix of rounding-constant and exact
    # K-tiles), bit for bit against the oracle; the two-workgroup 128 x 128
    # config, 64-bit sums by the 32-bit schedule plus redo (Q16) and by the
    # one-wave-per-SIMD exact kernel over the whole K (Q24: f > 20)
    g = torch.Generator("cpu").manual_seed(M + bits)
    K, N = 4096, 640
    a = _dyadic((M, K), -4, 4, -7, g, dtype)
    b = _dyadic((K, N), -4, 4, 0, g, dtype)
    a[M // 3: M // 3 + 40, 1024:1152] *= 64
    want = _oracle(a, b, None, bits, frac)
    got = _run(a, b, bits=bits, frac=frac, b_layout="nk")
    assert torch.equal(got, want), mismatch_report(got, want)
    got_kn = _run(a, b, bits=bits, frac=frac, b_layout="kn")
    assert torch.equal(got_kn, want), mismatch_report(got_kn, want)


def _lm_head_inputs(M, N, K, seed, dtype=torch.bfloat16, b_std=0.02):
    """A ~ N(0,1) [M, K] from a CPU generator; the weight ~ N(0, b_std) as vLLM
    stores it, [N, K], generated on the device (0.5-1 GB)."""
    g = torch.Generator("cpu").manual_seed(seed)
    a = torch.randn(M, K, generator=g).to(dtype)
    gd = torch.Generator(DEV).manual_seed(seed + 1)
    w = (torch.randn(N, K, generator=gd, device=DEV) * b_std).to(dtype)
    return a, w


@pytest.mark.parametrize("bits", [32, 64])
def test_lm_head_headline_m8192(bits):
    # BASELINE config 3 at the bench's M = 8192 (K = 4096, N = 128256): the
    # rows of the M = 8192 launch equal the same rows computed at M = 1, 32,
    # 256 and 2048 (skinny and large-M tiles), a split
    # launch gives the same bits, and a row x column block is within 1e-2 of
    # the oracle
    K, N, M = 4096, 128256, 8192
    a, w = _lm_head_inputs(M, N, K, seed=bits)
    ad, bd = a.to(DEV), w.t()
    full = KG.gemm_fxp_run(ad, bd, None, bits, 16)
    for m in (1, 32, 256, 2048):
        part = KG.gemm_fxp_run(ad[:m].contiguous(), bd, None, bits, 16)
        assert torch.equal(part, full[:m]), m
    last = KG.gemm_fxp_run(ad[M - 1:].contiguous(), bd, None, bits, 16)
    assert torch.equal(last[0], full[M - 1])
    assert torch.equal(KG.gemm_fxp_run(ad, bd, None, bits, 16, split_k=2), full)
    g = torch.Generator("cpu").manual_seed(3)
    rows = torch.randperm(M, generator=g)[:48]
    cols = torch.randperm(N, generator=g)[:1536]
    want = _oracle(a[rows], w[cols.to(DEV)].cpu().t().contiguous(), None, bits, 16)
    report = close_report(full[rows.to(DEV)][:, cols.to(DEV)], want)
    assert not report, report


@pytest.mark.parametrize("bits", [32, 64])
def test_lm_head_headline_exact_rows(bits):
    # the same launch shape on dyadic inputs (exact tile dots): 16 sampled
    # rows over all 128256 columns equal the oracle bit for bit
    K, N, M = 4096, 128256, 8192
    g = torch.Generator("cpu").manual_seed(40 + bits)
    a = _dyadic((M, K), -4, 4, -7, g, torch.bfloat16)
    gd = torch.Generator(DEV).manual_seed(41 + bits)
    w = (torch.randint(-4, 5, (N, K), generator=gd, device=DEV).to(torch.bfloat16))
    full = KG.gemm_fxp_run(a.to(DEV), w.t(), None, bits, 16)
    rows = torch.randperm(M, generator=g)[:16]
    want = _oracle(a[rows], w.cpu().t().contiguous(), None, bits, 16)
    got = full[rows.to(DEV)].cpu()
    assert torch.equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("M", [2048, 8192])
def test_gemm_config3prime_f16_f32(dtype, M):
    # BASELINE config 3': f16 and fp32 inputs, K = 4096, N = 14336, Q16.16 in
    # int32: rows equal the same rows at M = 1 and 32, split invariance, and
    # a row x column block within 1e-2 of the oracle
    K, N = 4096, 14336
    a, w = _lm_head_inputs(M, N, K, seed=M + 7, dtype=dtype)
    ad, bd = a.to(DEV), w.t()
    full = KG.gemm_fxp_run(ad, bd, None, 32, 16)
    for m in (1, 32):
        assert torch.equal(KG.gemm_fxp_run(ad[:m].contiguous(), bd, None, 32, 16), full[:m]), m
    assert torch.equal(KG.gemm_fxp_run(ad, bd, None, 32, 16, split_k=3), full)
    g = torch.Generator("cpu").manual_seed(M)
    rows = torch.randperm(M, generator=g)[:64]
    cols = torch.randperm(N, generator=g)[:1024]
    want = _oracle(a[rows], w[cols.to(DEV)].cpu().t().contiguous(), None, 32, 16)
    report = close_report(full[rows.to(DEV)][:, cols.to(DEV)], want)
    assert not report, report
