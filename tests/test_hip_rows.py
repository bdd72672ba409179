"""GPU parity: fixed_row_sum, RMSNorm(+residual), log-softmax vs the oracle.

Bit-exact against the oracle on seeded inputs (ragged, tiny, wider than the
register cache, misaligned), the reference's own RMSNorm tolerance and
permutation tests (fxpr_vllm/_tests/test_rms_norm.py) and sum tests
(fxpr_vllm/_tests/test_sum.py) restated, batch invariance, and run-to-run
identity.
"""

from __future__ import annotations

import ctypes
import json
import math
import pathlib

import numpy as np
import pytest
import torch

import fxpr_vllm  # noqa: F401
from fxpr_vllm import _hip
from fxpr_vllm import config as fxpr_config
from fxpr_vllm._kernels import rows as K
from oracle import numerics as N
from oracle import rows as R
from tests._util import IO_NAME, from_np, mismatch_report, nan_aware_equal, seeded, to_np

pytestmark = pytest.mark.gpu
KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())
DEV = "cuda"


# --------------------------------------------------------------------------
# fixed_row_sum


@pytest.mark.parametrize("qdtype", [torch.int16, torch.int32, torch.int64])
@pytest.mark.parametrize("b", [16, 32, 64])
@pytest.mark.parametrize("shape", [(7, 1000), (1, 100_003), (300, 3), (5,)])
def test_row_sum_bit_exact(qdtype, b, shape):
    info = torch.iinfo(qdtype)
    g = torch.Generator("cpu").manual_seed(b)
    q = torch.randint(info.min, info.max, shape, generator=g, dtype=qdtype)
    got = torch.ops.fxpr.fixed_row_sum(q.to(DEV), b).cpu()
    want = N.fixed_row_sum(q.numpy(), b)
    assert got.shape == tuple(shape[:-1])
    assert np.array_equal(got.numpy(), want)


def test_row_sum_reference_kats():
    # fxpr_vllm/_tests/test_sum.py:50-119 through float_to_fixed + fixed_row_sum
    k = KATS["sum_on_q_grid"]
    q = torch.tensor(k["q_i32"], dtype=torch.int32, device=DEV)
    x = torch.ops.fxpr.fixed_to_float(q.to(torch.int64), 32, 16)
    s = torch.ops.fxpr.fixed_row_sum(torch.ops.fxpr.float_to_fixed(x, 32, 16), 32)
    assert s.item() == k["sum_q"]
    assert torch.equal(x.sum().reshape(1).view(torch.int32).cpu(),
                       torch.ops.fxpr.fixed_to_float(s.to(torch.int64), 32, 16).reshape(1).view(torch.int32).cpu())
    for name in ("sum_saturates_max", "sum_saturates_min"):
        k = KATS[name]
        q = torch.ops.fxpr.float_to_fixed(torch.tensor(k["x_f32"], device=DEV), 32, 16)
        assert torch.ops.fxpr.fixed_row_sum(q, 32).item() == k["sum_q"]
    k = KATS["sum_associativity"]
    a = torch.ops.fxpr.fixed_row_sum(torch.ops.fxpr.float_to_fixed(torch.tensor(k["order_a"], device=DEV), 64, 16), 64)
    b = torch.ops.fxpr.fixed_row_sum(torch.ops.fxpr.float_to_fixed(torch.tensor(k["order_b"], device=DEV), 64, 16), 64)
    assert a.item() == b.item()
    assert torch.ops.fxpr.fixed_to_float(a, 32, 16).item() == k["sum_f32"]


def test_row_sum_empty():
    assert torch.ops.fxpr.fixed_row_sum(torch.empty(3, 0, dtype=torch.int32, device=DEV), 32).tolist() == [0, 0, 0]
    assert torch.ops.fxpr.fixed_row_sum(torch.empty(0, 4, dtype=torch.int32, device=DEV), 32).shape == (0,)


# --------------------------------------------------------------------------
# RMSNorm


def _rms_case(io_dtype, shape, seed, residual):
    x = seeded(shape, seed, dtype=io_dtype)
    w = seeded(shape[-1:], seed + 1, std=0.1, mean=1.0, dtype=io_dtype)
    r = seeded(shape, seed + 2, dtype=io_dtype) if residual else None
    return x, w, r


def _rms_check(x, w, r, eps=1e-6):
    io = IO_NAME[x.dtype]
    xd, wd = x.to(DEV), w.to(DEV)
    rd = r.to(DEV).clone() if r is not None else None
    if rd is None:
        y = K.rms_norm_fxp_run(xd, wd, eps)
    else:
        y = K.rms_norm_fxp_residual_run(xd, rd, wd, eps)
    y_want, r_want = R.rms_norm(to_np(x), to_np(w), eps, io, residual=None if r is None else to_np(r))
    y_want = from_np(y_want, x.dtype)
    assert nan_aware_equal(y.cpu(), y_want), mismatch_report(y.cpu(), y_want)
    if r is not None:
        r_want = from_np(r_want, x.dtype)
        assert nan_aware_equal(rd.cpu(), r_want), mismatch_report(rd.cpu(), r_want)
    return y, rd


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("residual", [False, True])
@pytest.mark.parametrize("scale", [1.0, 30.0])
@pytest.mark.parametrize("shape", [(64, 4096), (3, 7), (1, 1), (2, 40_000), (17, 1000)])
def test_rms_norm_bit_exact(dtype, residual, scale, shape):
    # (2, 40000) is longer than the register cache: its tail is re-read and
    # its residual written back in the sum pass
    x, w, r = _rms_case(dtype, shape, seed=shape[-1] % 1000, residual=residual)
    x = (x.float() * scale).to(dtype)
    _rms_check(x, w, r)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("residual", [False, True])
def test_rms_norm_scalar_path_many_elements(dtype, residual):
    # a hidden size that is not a multiple of 8 takes the one-element-per-lane
    # kernel; 262K outputs put dozens of fp32 results on an f16 rounding
    # midpoint, where converting the fp32 product (what the oracle does)
    # differs from rounding the exact product x * inv * w to f16 in one step
    x, w, r = _rms_case(dtype, (64, 4099), seed=23, residual=residual)
    _rms_check(x, w, r)


def _realistic_rows(H=4096, seed=0):
    """RMS 3, 5, 20, 100, 1e4 and 1e-3 rows, plus an N(0, 0.5) row with one
    channel at 1500 (residual-stream magnitudes where a Q16.16 int32 sum of
    squares would saturate)."""
    g = torch.Generator("cpu").manual_seed(seed)
    rows = [torch.randn(H, generator=g) * s for s in (3.0, 5.0, 20.0, 100.0, 1.0e4, 1.0e-3)]
    spike = torch.randn(H, generator=g) * 0.5
    spike[H // 3] = 1500.0
    return torch.stack(rows + [spike])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("residual", [False, True])
def test_rms_norm_realistic_magnitudes(dtype, residual):
    # bit-exact vs the oracle, and within the reference's own tolerances
    # (fxpr_vllm/_tests/test_rms_norm.py: 2e-2 bf16, 5e-3 f16, 5e-4 fp32) of
    # the reference's fp32 RMSNorm (_triton/rms_norm.py:38-64)
    x = _realistic_rows().to(dtype)
    r = (_realistic_rows(seed=1) * 0.5).to(dtype) if residual else None
    w = seeded((4096,), 7, std=0.1, mean=1.0, dtype=dtype)
    y, rd = _rms_check(x, w, r)
    v = x.double() + (r.double() if residual else 0.0)
    u = rd.cpu().double() if residual else x.double()
    ref = u * w.double() / torch.sqrt((v * v).mean(-1, keepdim=True) + 1e-6)
    ref = ref.float().to(dtype).double()
    tol = _TOL[dtype]
    assert torch.allclose(y.cpu().double(), ref, atol=tol, rtol=tol)


def test_rms_norm_special_rows():
    # zero, subnormal, subnormal mean square, fp32-overflowing mean square,
    # inf and NaN rows (eps 1e-6 and 0)
    H = 64
    x = torch.zeros(6, H)
    x[1] = 2.0 ** -140
    x[2] = 2.0 ** -70
    x[3] = 1.0e30
    x[4, 0], x[4, 1:] = float("inf"), 1.0
    x[5, 0], x[5, 1:] = float("nan"), 1.0
    w = torch.full((H,), 2.0)
    for eps in (1e-6, 0.0):
        for rows in (x, x.repeat(1, 1000)[:, : H * 1000]):
            ww = w.repeat(rows.shape[1] // H)
            _rms_check(rows, ww, None, eps=eps)
            _rms_check(rows, ww, torch.zeros_like(rows), eps=eps)


def test_rms_norm_ignores_fixed_point_knobs(monkeypatch):
    # like the reference's RMSNorm, the op takes no fixed-point format: the
    # FXPR_* knobs (which the GEMM and attention read) do not change its bits
    x, w, r = _rms_case(torch.bfloat16, (8, 4096), 5, True)
    outs = []
    for b, f in ((32, 16), (64, 32), (16, 8)):
        monkeypatch.setenv("FXPR_INT_BITS", str(b))
        monkeypatch.setenv("FXPR_FRAC_BITS", str(f))
        fxpr_config.reset_runtime_config()
        try:
            rd = r.to(DEV).clone()
            y = torch.ops.fxpr.rms_norm_fxp_residual(x.to(DEV), rd, w.to(DEV), 1e-6)
            y2 = torch.ops.fxpr.rms_norm_fxp(x.to(DEV), w.to(DEV), 1e-6)
            outs.append((y.cpu(), rd.cpu(), y2.cpu()))
        finally:
            fxpr_config.reset_runtime_config()
    y_want, r_want = R.rms_norm(to_np(x), to_np(w), 1e-6, "bf16", residual=to_np(r))
    y2_want, _ = R.rms_norm(to_np(x), to_np(w), 1e-6, "bf16")
    for y, rd, y2 in outs:
        assert torch.equal(y, from_np(y_want, torch.bfloat16))
        assert torch.equal(rd, from_np(r_want, torch.bfloat16))
        assert torch.equal(y2, from_np(y2_want, torch.bfloat16))


def test_rms_norm_noncontiguous_residual_copy_back():
    x, w, _ = _rms_case(torch.float16, (6, 64), 9, False)
    base = seeded((64, 6), 10, dtype=torch.float16)
    r_nc = base.to(DEV).t()  # [6, 64] non-contiguous view
    r_host = base.t().contiguous()
    y = torch.ops.fxpr.rms_norm_fxp_residual(x.to(DEV), r_nc, w.to(DEV), 1e-6)
    y_want, r_want = R.rms_norm(to_np(x), to_np(w), 1e-6, "f16", residual=to_np(r_host))
    assert torch.equal(y.cpu(), from_np(y_want, torch.float16))
    assert torch.equal(r_nc.cpu(), from_np(r_want, torch.float16))


def test_rms_norm_batch_invariance():
    x, w, r = _rms_case(torch.bfloat16, (128, 4096), 21, True)
    xd, wd = x.to(DEV), w.to(DEV)
    full = K.rms_norm_fxp_run(xd, wd, 1e-6)
    for row in (0, 3, 17, 64, 127):
        for batch in (1, 4, 16, 128):
            if row >= batch:
                continue
            sub = xd[:batch].clone()
            out = K.rms_norm_fxp_run(sub, wd, 1e-6)
            assert torch.equal(out[row], full[row])


@pytest.mark.parametrize("shape", [(2, 7), (3, 16), (4, 31)])
def test_reference_rms_norm_correctness(shape):
    # fxpr_vllm/_tests/test_rms_norm.py:39-57
    g = torch.Generator("cpu").manual_seed(0)
    x = ((torch.rand(shape, generator=g) - 0.5) * 32.0).to(DEV)
    w = ((torch.rand(shape[1:], generator=g) - 0.5) * 4.0).to(DEV)
    got = torch.ops.fxpr.rms_norm_fxp(x, w, 1e-6)
    ref = x * w * (1.0 / torch.sqrt((x * x).mean(dim=-1, keepdim=True) + 1e-6))
    assert torch.allclose(got, ref, atol=5e-4, rtol=5e-4)


_TOL = {torch.float32: 5e-4, torch.float16: 5e-3, torch.bfloat16: 2e-2}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_reference_rms_norm_residual_native_dtype(dtype):
    # fxpr_vllm/_tests/test_rms_norm.py:100-130
    g = torch.Generator("cpu").manual_seed(11)
    x = ((torch.rand((4, 32), generator=g) - 0.5) * 2.0).to(dtype).to(DEV)
    r = ((torch.rand((4, 32), generator=g) - 0.5) * 2.0).to(dtype).to(DEV)
    w = ((torch.rand((32,), generator=g) - 0.5) * 2.0).to(dtype).to(DEV)
    r_orig = r.clone()
    out = torch.ops.fxpr.rms_norm_fxp_residual(x, r, w, 1e-6)
    assert out.dtype == dtype and r.dtype == dtype
    expected_r = (x.float() + r_orig.float()).to(dtype)
    tol = _TOL[dtype]
    assert torch.allclose(r.float(), expected_r.float(), atol=tol, rtol=tol)


def test_reference_rms_norm_associativity():
    # fxpr_vllm/_tests/test_rms_norm.py:133-151
    k = KATS["rms_norm_associativity"]
    xa = torch.tensor(k["x_f32"], device=DEV)
    perm = torch.tensor(k["perm"], device=DEV)
    x = torch.stack([xa, xa[perm]])
    y = torch.ops.fxpr.rms_norm_fxp(x, torch.ones(5, device=DEV), k["eps"])
    assert torch.equal(y[1], y[0][perm])


def test_rms_norm_errors_and_empty():
    x = torch.ones(2, 8, device=DEV)
    with pytest.raises(TypeError):
        torch.ops.fxpr.rms_norm_fxp(x, torch.ones(8, device=DEV, dtype=torch.float16), 1e-6)
    with pytest.raises(TypeError):
        torch.ops.fxpr.rms_norm_fxp(x.double(), torch.ones(8, device=DEV).double(), 1e-6)
    with pytest.raises(ValueError):
        torch.ops.fxpr.rms_norm_fxp_residual(x, torch.ones(3, 8, device=DEV), torch.ones(8, device=DEV), 1e-6)
    e = torch.ops.fxpr.rms_norm_fxp(torch.empty(0, 8, device=DEV), torch.ones(8, device=DEV), 1e-6)
    assert e.shape == (0, 8)


def test_rms_norm_run_to_run():
    x, w, _ = _rms_case(torch.bfloat16, (512, 4096), 31, False)
    xd, wd = x.to(DEV), w.to(DEV)
    a = torch.ops.fxpr.rms_norm_fxp(xd, wd, 1e-6)
    for _ in range(3):
        assert torch.equal(a, torch.ops.fxpr.rms_norm_fxp(xd, wd, 1e-6))


# --------------------------------------------------------------------------
# log-softmax


def _logits(rows, vocab, seed, dtype=torch.bfloat16):
    """~N(0, 4^2) with 1% outliers at +-30 (the bandwidth config's data)."""
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(rows, vocab, generator=g) * 4.0
    mask = torch.rand(rows, vocab, generator=g) < 0.01
    sign = torch.where(torch.rand(rows, vocab, generator=g) < 0.5, -1.0, 1.0)
    x = torch.where(mask, 30.0 * sign, x)
    return x.to(dtype)


@pytest.mark.parametrize("b,f", [(32, 16), (64, 32), (16, 8)])
@pytest.mark.parametrize("out_dtype", [None, torch.float32])
def test_log_softmax_vocab_bit_exact(b, f, out_dtype):
    x = _logits(4, 128_256, seed=b + f)
    got = torch.ops.fxpr.log_softmax_fxp(x.to(DEV), b, f, out_dtype).cpu()
    want = from_np(R.log_softmax(to_np(x), "bf16", IO_NAME[out_dtype or x.dtype], b, f), out_dtype or x.dtype)
    assert nan_aware_equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 1), (5, 7), (3, 1000), (2, 300_001), (33, 4096)])
def test_log_softmax_shapes_bit_exact(dtype, shape):
    x = _logits(*shape, seed=shape[1], dtype=dtype)
    got = torch.ops.fxpr.log_softmax_fxp(x.to(DEV), 32, 16).cpu()
    want = from_np(R.log_softmax(to_np(x), IO_NAME[dtype], IO_NAME[dtype], 32, 16), dtype)
    assert nan_aware_equal(got, want), mismatch_report(got, want)


def test_log_softmax_special_rows():
    x = torch.tensor([[-float("inf")] * 8, [float("nan"), 0, 1, 2, 3, 4, 5, 6],
                      [0, -float("inf"), 1, -float("inf"), 2, 3, 4, 5]], dtype=torch.float32)
    got = torch.ops.fxpr.log_softmax_fxp(x.to(DEV), 32, 16).cpu()
    want = torch.from_numpy(R.log_softmax(x.numpy(), "f32", "f32", 32, 16))
    assert nan_aware_equal(got, want)


@pytest.mark.parametrize("b,f", [(32, 16), (16, 8), (16, 16), (32, 32)])
def test_log_softmax_wide_sums_and_exact_path(b, f):
    # flat rows whose denominator V * 2^f exceeds the term width (the sum is
    # exact and unclamped), next to ordinary rows; (16, 16) and (32, 32) take
    # the exact per-term path (a term can exceed the rounding constant's range
    # or qmax), (32, 16) and (16, 8) the rounding-constant one with 32-bit
    # lane sums
    x = _logits(6, 128_256, seed=b * f)
    x[0] = 0.0
    x[1] = -3.5
    x[2, :64_000] = 7.0
    got = torch.ops.fxpr.log_softmax_fxp(x.to(DEV), b, f).cpu()
    want = from_np(R.log_softmax(to_np(x), "bf16", "bf16", b, f), x.dtype)
    assert nan_aware_equal(got, want), mismatch_report(got, want)


def test_log_softmax_close_to_torch():
    x = _logits(16, 32_000, seed=4, dtype=torch.float32)
    got = torch.ops.fxpr.log_softmax_fxp(x.to(DEV), 64, 32).cpu()
    ref = torch.log_softmax(x.double(), dim=-1)
    assert torch.allclose(got.double(), ref, atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("b,f", [(32, 16), (16, 8), (64, 32), (64, 63), (32, 0)])
def test_log_softmax_flat_full_vocab_row(b, f):
    # a flat [V = 128256] row: V * 2^f exceeds the knob's width, the exact
    # denominator does not saturate (128-bit for (64, 63)), y = -ln V
    V = 128_256
    x = torch.zeros(3, V, dtype=torch.bfloat16)
    x[1] = 5.0
    x[2, : V // 2] = -1.0
    # the launcher (the op admits frac bits 8 / 16 / 32 only, fxpr_vllm/_lib.py:55-56)
    for out_dtype in (None, torch.float32):
        got = K.log_softmax_fxp_run(x.to(DEV), b, f, out_dtype).cpu()
        want = from_np(R.log_softmax(to_np(x), "bf16", IO_NAME[out_dtype or x.dtype], b, f), out_dtype or x.dtype)
        assert nan_aware_equal(got, want), mismatch_report(got, want)
    got = K.log_softmax_fxp_run(x.to(DEV), b, f, torch.float32).cpu()
    assert abs(got[0, 0].item() + math.log(V)) < 4e-6 * math.log(V)
    assert abs(got[1, 0].item() + math.log(V)) < 4e-6 * math.log(V)
    # the exp of the output sums to 1 up to the quantisation of the terms
    # (each term is off by at most 2^-(f+1) of the row maximum's weight)
    if f >= 16:
        assert abs(torch.exp(got.double()).sum(-1) - 1).max().item() < V * 2.0 ** -(f + 1) + 1e-5


def test_log_softmax_split_rows_equal_one_workgroup_rows():
    # up to 1024 rows of at least 4096 16-byte vectors are shared by 2..16
    # workgroups each (span maxima and exact span sums exchanged through
    # device memory); 1025 rows take one workgroup per row: same bits
    x = _logits(1025, 32_768, seed=11).to(DEV)
    for b, f in ((32, 16), (64, 32)):
        one = torch.ops.fxpr.log_softmax_fxp(x, b, f)
        split = torch.ops.fxpr.log_softmax_fxp(x[:1024].clone(), b, f)
        assert torch.equal(split, one[:1024]), (b, f)


@pytest.mark.parametrize("cols,dtype,out_dtype,b,f", [
    (32_768, torch.bfloat16, None, 32, 16),           # 2 spans of 2048 vectors
    (40_000, torch.float16, torch.float32, 16, 8),    # 4 ragged spans
    (128_256, torch.bfloat16, torch.float32, 64, 32),  # 8 spans, exact per-term path
    (262_144, torch.bfloat16, None, 32, 16),          # 16 spans
    (100_000, torch.float32, None, 64, 32),           # f32 rows, 16 ragged spans
])
def test_log_softmax_split_counts_bit_exact(cols, dtype, out_dtype, b, f):
    x = _logits(3, cols, seed=cols % 97, dtype=dtype)
    x[1, cols // 3] = 80.0  # the maximum inside one span: the others hold only small terms
    got = torch.ops.fxpr.log_softmax_fxp(x.to(DEV), b, f, out_dtype).cpu()
    want = from_np(R.log_softmax(to_np(x), IO_NAME[dtype], IO_NAME[out_dtype or dtype], b, f),
                   out_dtype or dtype)
    assert nan_aware_equal(got, want), mismatch_report(got, want)


def test_log_softmax_split_concurrent_streams():
    # every stream has its own sync region (16 per device; later streams take
    # the one-workgroup kernel): concurrent calls on 20 streams, each checked
    # against a serial call
    xs = [_logits(8, 128_256, seed=40 + i).to(DEV) for i in range(20)]
    want = [torch.ops.fxpr.log_softmax_fxp(x, 32, 16) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in xs]
    outs = []
    for _ in range(3):
        for s, x in zip(streams, xs):
            with torch.cuda.stream(s):
                outs.append(torch.ops.fxpr.log_softmax_fxp(x, 32, 16))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, want[i % len(xs)]), i


def _lsm_fallbacks() -> int:
    n = ctypes.c_ulonglong(0)
    _hip.call("fxpr_debug_lsm_fallbacks", ctypes.byref(n))
    return n.value


@pytest.mark.parametrize("max_tries,sum_tries", [(0, None), (None, 0)])
def test_log_softmax_split_giveup_paths_bit_exact(max_tries, sum_tries):
    # The split kernel's polls are bounded. The host sets a poll's limit to 0
    # tries, so every workgroup gives up at once and computes what it waited
    # for from the input (the row maximum and exact sum, or the exact sum
    # after its own span sum was published): the bits equal the oracle's and
    # every kernel exits normally. A normal launch on the same stream right
    # after must find consistent sync state (its generation advanced by the
    # last span of each row) and give the same bits again.
    lib = _hip.load()
    default = lib.fxpr_debug_lsm_default_spin_limit()
    rows, cols = 3, 128_256                    # 8 spans of 2004 vectors per row
    x = _logits(rows, cols, seed=23)
    x[2, 77_000] = 75.0
    want = from_np(R.log_softmax(to_np(x), "bf16", "f32", 32, 16), torch.float32)
    xd = x.to(DEV)
    torch.cuda.synchronize()
    before = _lsm_fallbacks()
    _hip.call("fxpr_debug_set_lsm_spin_limit", default if max_tries is None else max_tries,
              default if sum_tries is None else sum_tries)
    try:
        got = torch.ops.fxpr.log_softmax_fxp(xd, 32, 16, torch.float32)
        torch.cuda.synchronize()
    finally:
        _hip.call("fxpr_debug_set_lsm_spin_limit", default, default)
    assert _lsm_fallbacks() - before == rows * 8   # every span took the path
    assert nan_aware_equal(got.cpu(), want), mismatch_report(got.cpu(), want)
    again = torch.ops.fxpr.log_softmax_fxp(xd, 32, 16, torch.float32)
    torch.cuda.synchronize()
    assert _lsm_fallbacks() - before == rows * 8
    assert torch.equal(again, got)


def test_log_softmax_batch_and_run_invariance():
    x = _logits(64, 128_256, seed=8).to(DEV)
    full = torch.ops.fxpr.log_softmax_fxp(x, 32, 16)
    for row in (0, 5, 63):
        assert torch.equal(torch.ops.fxpr.log_softmax_fxp(x[row:row + 1].clone(), 32, 16)[0], full[row])
    assert torch.equal(full, torch.ops.fxpr.log_softmax_fxp(x, 32, 16))


def test_rms_norm_rrms_correctly_rounded():
    # 20k rows, each a different constant: every row exercises one IEEE
    # sqrt + division on the device; a non-correctly-rounded sqrt or
    # division shows up as ulp differences against the oracle
    g = torch.Generator("cpu").manual_seed(123)
    c = torch.exp(torch.rand(20_000, generator=g) * 12 - 6)
    x = c[:, None].expand(20_000, 64).contiguous()
    w = torch.ones(64)
    y = K.rms_norm_fxp_run(x.to(DEV), w.to(DEV), 1e-6).cpu()
    want = torch.from_numpy(R.rms_norm(x.numpy(), w.numpy(), 1e-6, "f32")[0])
    assert torch.equal(y, want), mismatch_report(y, want)


@pytest.mark.parametrize("b", [32, 64])
def test_config1_plumbing_full_shape(b):
    # fp32 x [4096, 4096] ~ N(0,1), residual ~ N(0,1),
    # weight ~ N(1, 0.1), eps 1e-6, seed 0; float_to_fixed -> fixed_row_sum ->
    # fixed_to_float at Q16.16 in int32 / int64, and RMSNorm (+ residual),
    # all bit for bit against the oracle
    g = torch.Generator("cpu").manual_seed(0)
    x = torch.randn(4096, 4096, generator=g)
    r = torch.randn(4096, 4096, generator=g)
    w = torch.randn(4096, generator=g) * 0.1 + 1.0
    xd = x.to(DEV)
    q = torch.ops.fxpr.float_to_fixed(xd, b, 16)
    s = torch.ops.fxpr.fixed_row_sum(q, b)
    y = torch.ops.fxpr.fixed_to_float(s, 32, 16)
    q_want = N.float_to_fixed(x.numpy(), b, 16)
    assert np.array_equal(q.cpu().numpy(), q_want)
    s_want = N.fixed_row_sum(q_want, b)
    assert np.array_equal(s.cpu().numpy(), s_want)
    assert np.array_equal(y.cpu().numpy(), N.fixed_to_float(s_want, 32, 16))
    if b == 32:
        y, _ = _rms_check(x, w, None)
        _rms_check(x, w, r)
        ref = x.double() * w.double() / torch.sqrt((x.double() ** 2).mean(-1, keepdim=True) + 1e-6)
        assert torch.allclose(y.cpu().double(), ref, atol=5e-4, rtol=5e-4)
