"""GPU parity: float_to_fixed / fixed_to_float vs the oracle, bit for bit.

Restates the reference's cast tests (fxpr_vllm/_tests/test_fixed_point_cast.py)
on the HIP path and extends them to every fp16 bit pattern, stratified fp32
(ties, subnormals, +-inf, NaN, saturation edges), fp64 inputs, every
(int_bits, frac_bits) pair the schema accepts, ragged and misaligned sizes.
"""

from __future__ import annotations

import json
import pathlib

import numpy as np
import pytest
import torch

import fxpr_vllm  # noqa: F401
from oracle import numerics as N
from tests._util import to_np
from tests.test_oracle_numerics import all_f16, stratified_f32

pytestmark = pytest.mark.gpu
KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())
DEV = "cuda"


def _inputs(dtype: torch.dtype) -> torch.Tensor:
    f16 = torch.from_numpy(all_f16().astype(np.float32))
    strat = torch.from_numpy(stratified_f32(seed=11, n=20000))
    g = torch.Generator("cpu").manual_seed(3)
    big = torch.randn(1_000_003, generator=g) * 300.0
    x = torch.cat([f16, strat, big])
    if dtype == torch.float16:
        x = x.to(torch.float16)
    elif dtype == torch.float64:
        x = x.double() * (1.0 + 2.0 ** -30)  # off the fp32 grid
    return x


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("b", [16, 32, 64])
@pytest.mark.parametrize("f", [8, 16, 32])
def test_float_to_fixed_bit_exact(dtype, b, f):
    x = _inputs(dtype)
    got = torch.ops.fxpr.float_to_fixed(x.to(DEV), b, f).cpu()
    want = N.float_to_fixed(to_np(x), b, f)
    assert got.dtype == {16: torch.int16, 32: torch.int32, 64: torch.int64}[b]
    assert np.array_equal(got.numpy(), want)


def test_float_to_fixed_misaligned_and_noncontiguous():
    x = _inputs(torch.float32)[:100_001]
    xd = x.to(DEV)
    for view, ref in ((xd[1:], x[1:]), (xd[3:-2], x[3:-2]), (xd[::3], x[::3])):
        got = torch.ops.fxpr.float_to_fixed(view, 32, 16).cpu()
        assert np.array_equal(got.numpy(), N.float_to_fixed(ref.numpy(), 32, 16))
    x2 = torch.randn(64, 33).to(DEV).t()  # non-contiguous 2-D
    got = torch.ops.fxpr.float_to_fixed(x2, 64, 32)
    assert got.shape == x2.shape and got.is_contiguous()
    assert np.array_equal(got.cpu().numpy(), N.float_to_fixed(x2.cpu().numpy(), 64, 32))


@pytest.mark.parametrize("qdtype", [torch.int16, torch.int32, torch.int64])
@pytest.mark.parametrize("fb", [16, 32, 64])
@pytest.mark.parametrize("f", [8, 16, 32])
def test_fixed_to_float_bit_exact(qdtype, fb, f):
    info = torch.iinfo(qdtype)
    g = torch.Generator("cpu").manual_seed(fb + f)
    if qdtype == torch.int16:
        q = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    else:
        rnd = torch.randint(info.min, info.max, (200_001,), generator=g, dtype=qdtype)
        small = torch.randint(-(1 << 20), 1 << 20, (5000,), generator=g, dtype=qdtype)
        edge = torch.tensor([0, 1, -1, info.max, info.min, info.max - 1, info.min + 1,
                             (1 << 24) + 1, -((1 << 24) + 1)], dtype=qdtype)
        q = torch.cat([edge, small, rnd])
    got = torch.ops.fxpr.fixed_to_float(q.to(DEV), fb, f).cpu()
    want = N.fixed_to_float(q.numpy(), fb, f)
    assert got.dtype == {16: torch.float16, 32: torch.float32, 64: torch.float64}[fb]
    assert np.array_equal(got.numpy().view(np.uint8), want.view(np.uint8))


def test_reference_cast_known_values():
    # fxpr_vllm/_tests/test_fixed_point_cast.py:7-42
    k = KATS["cast_known_values"]
    x = torch.tensor(k["x_f32"], device=DEV)
    got = torch.ops.fxpr.float_to_fixed(x, 32, 16)
    assert torch.equal(got.cpu(), torch.tensor(k["q_i32"], dtype=torch.int32))


def test_reference_cast_saturation_and_roundtrips():
    k = KATS["cast_saturation"]
    got = torch.ops.fxpr.float_to_fixed(torch.tensor(k["x_f32"], device=DEV), 32, 16).cpu().tolist()
    for v, (lo, hi) in zip(got, k["q_bounds"]):
        assert lo <= v <= hi
    k = KATS["float_roundtrip_lossless"]
    base = torch.tensor(k["x_f32"], device=DEV)
    back = torch.ops.fxpr.fixed_to_float(torch.ops.fxpr.float_to_fixed(base, 32, 16), 32, 16)
    assert torch.equal(back, base)
    k = KATS["fixed_roundtrip_lossless"]
    q = torch.tensor(k["q_i32"], dtype=torch.int32, device=DEV)
    assert torch.equal(torch.ops.fxpr.float_to_fixed(torch.ops.fxpr.fixed_to_float(q, 32, 16), 32, 16), q)
    k = KATS["float_roundtrip_frac_bits"]
    base = torch.tensor(k["x_f32"], device=DEV)
    for f in k["frac_bits"]:
        q = torch.ops.fxpr.float_to_fixed(base, 64, f)
        assert torch.equal(torch.ops.fxpr.fixed_to_float(q, 32, f), base)


def test_cast_errors_and_empty():
    with pytest.raises(TypeError):
        torch.ops.fxpr.float_to_fixed(torch.ones(4, device=DEV, dtype=torch.bfloat16), 32, 16)
    with pytest.raises(TypeError):
        torch.ops.fxpr.fixed_to_float(torch.ones(4, device=DEV), 32, 16)
    with pytest.raises(ValueError):
        torch.ops.fxpr.float_to_fixed(torch.ones(4, device=DEV), 24, 16)
    with pytest.raises(ValueError):
        torch.ops.fxpr.float_to_fixed(torch.ones(4, device=DEV), 32, 12)
    e = torch.ops.fxpr.float_to_fixed(torch.empty(0, 5, device=DEV), 32, 16)
    assert e.shape == (0, 5) and e.dtype == torch.int32
    e = torch.ops.fxpr.fixed_to_float(torch.empty(0, device=DEV, dtype=torch.int64), 16, 16)
    assert e.shape == (0,) and e.dtype == torch.float16


def test_casts_run_to_run_identical():
    x = _inputs(torch.float32).to(DEV)
    a = torch.ops.fxpr.float_to_fixed(x, 32, 16)
    for _ in range(3):
        assert torch.equal(a, torch.ops.fxpr.float_to_fixed(x, 32, 16))
