"""Elementwise float <-> fixed-point casts (launchers for csrc/casts.hip).

Same dtype rules, contiguity, empty handling and error classes as the
reference launchers (fxpr_vllm/_triton/casts.py:14-18, 57-126).
"""

from __future__ import annotations

import torch

from .. import _hip
from .fxp import fxp_constants

_SUPPORTED_FLOAT_DTYPES = (torch.float16, torch.float32, torch.float64)
_SUPPORTED_INT_DTYPES = (torch.int16, torch.int32, torch.int64)
_FLOAT_BITS_TO_TORCH = {16: torch.float16, 32: torch.float32, 64: torch.float64}


def float_to_fixed_run(x: torch.Tensor, int_bits: int, fxp_frac_bits: int) -> torch.Tensor:
    if not x.is_cuda:
        raise RuntimeError("float_to_fixed: input must be CUDA")
    if x.dtype not in _SUPPORTED_FLOAT_DTYPES:
        raise TypeError(
            f"float_to_fixed: unsupported input dtype {x.dtype}; "
            f"expected one of {_SUPPORTED_FLOAT_DTYPES}"
        )
    _, _, _, _, int_dtype = fxp_constants(int_bits, fxp_frac_bits)
    x_c = x.contiguous()
    y = torch.empty_like(x_c, dtype=int_dtype)
    n = x_c.numel()
    if n == 0:
        return y
    _hip.call(
        "fxpr_float_to_fixed", x_c.data_ptr(), _hip.DTYPE_CODE[x_c.dtype], y.data_ptr(),
        int(int_bits), int(fxp_frac_bits), n, _hip.stream_ptr(x_c.device),
    )
    return y


def fixed_to_float_run(x: torch.Tensor, float_bits: int, fxp_frac_bits: int) -> torch.Tensor:
    if not x.is_cuda:
        raise RuntimeError("fixed_to_float: input must be CUDA")
    if x.dtype not in _SUPPORTED_INT_DTYPES:
        raise TypeError(
            f"fixed_to_float: unsupported input dtype {x.dtype}; "
            f"expected one of {_SUPPORTED_INT_DTYPES}"
        )
    if float_bits not in _FLOAT_BITS_TO_TORCH:
        raise ValueError(f"float_bits must be 16/32/64, got {float_bits}")
    if not (0 <= fxp_frac_bits < 64):
        raise ValueError(f"fxp_frac_bits must satisfy 0 <= N < 64, got {fxp_frac_bits}")
    x_c = x.contiguous()
    y = torch.empty_like(x_c, dtype=_FLOAT_BITS_TO_TORCH[float_bits])
    n = x_c.numel()
    if n == 0:
        return y
    _hip.call(
        "fxpr_fixed_to_float", x_c.data_ptr(), _hip.DTYPE_CODE[x_c.dtype], y.data_ptr(),
        int(float_bits), int(fxp_frac_bits), n, _hip.stream_ptr(x_c.device),
    )
    return y
