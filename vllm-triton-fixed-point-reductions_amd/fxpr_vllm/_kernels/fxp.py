"""Host-side fixed-point constants (the device side is csrc/fxp_device.h)."""

from __future__ import annotations

import torch

_TORCH_INT_DTYPE_BY_BITS = {16: torch.int16, 32: torch.int32, 64: torch.int64}

_CONSTANTS_CACHE: dict[tuple[int, int], tuple] = {}


def fxp_constants(int_bits: int, frac_bits: int):
    """(scale, inv_scale, qmin, qmax, torch_int_dtype) for a Q format.

    Same validation and values as fxp_constants in the reference
    (fxpr_vllm/_triton/fxp.py:31-53): int_bits in {16, 32, 64} and
    0 <= frac_bits < 64, else ValueError. Memoised: launchers call it per op.
    """
    key = (int_bits, frac_bits)
    hit = _CONSTANTS_CACHE.get(key)
    if hit is not None:
        return hit
    if int_bits not in _TORCH_INT_DTYPE_BY_BITS:
        raise ValueError(f"int_bits must be 16/32/64, got {int_bits}")
    if not (0 <= frac_bits < 64):
        raise ValueError(f"frac_bits must satisfy 0 <= N < 64, got {frac_bits}")
    scale = float(1 << frac_bits)
    res = (
        scale,
        1.0 / scale,
        float(-(1 << (int_bits - 1))),
        float((1 << (int_bits - 1)) - 1),
        _TORCH_INT_DTYPE_BY_BITS[int_bits],
    )
    _CONSTANTS_CACHE[key] = res
    return res


def int_dtype_for_bits(int_bits: int) -> torch.dtype:
    try:
        return _TORCH_INT_DTYPE_BY_BITS[int(int_bits)]
    except KeyError:
        raise ValueError(f"int_bits must be 16/32/64, got {int_bits}") from None
