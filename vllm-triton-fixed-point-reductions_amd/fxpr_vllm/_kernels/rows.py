"""Row-reduction launchers: fixed-point row sum, RMSNorm(+residual), log-softmax
(csrc/rows.hip)."""

from __future__ import annotations

import math

import torch

from .. import _hip
from ..config import get_runtime_config
from .fxp import fxp_constants, int_dtype_for_bits

_SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_INT_DTYPES = (torch.int16, torch.int32, torch.int64)


def _bits(int_bits: int | None, frac_bits: int | None) -> tuple[int, int]:
    if int_bits is None or frac_bits is None:
        cfg = get_runtime_config()
        int_bits = cfg.fxp_int_bits if int_bits is None else int_bits
        frac_bits = cfg.fxp_frac_bits if frac_bits is None else frac_bits
    fxp_constants(int(int_bits), int(frac_bits))  # validates
    return int(int_bits), int(frac_bits)


def fixed_row_sum_run(q: torch.Tensor, int_bits: int) -> torch.Tensor:
    """Exact sum over the last dim, saturated once to int_bits.

    The reference does this with torch in its tests
    (fxpr_vllm/_tests/test_sum.py:12-16); here it is a kernel.
    """
    if not q.is_cuda:
        raise RuntimeError("fixed_row_sum: input must be CUDA")
    if q.dtype not in _INT_DTYPES:
        raise TypeError(f"fixed_row_sum: unsupported input dtype {q.dtype}; expected one of {_INT_DTYPES}")
    out_dtype = int_dtype_for_bits(int_bits)
    q_c = q.contiguous()
    out_shape = tuple(q_c.shape[:-1]) if q_c.dim() else ()
    cols = q_c.shape[-1] if q_c.dim() else 1
    rows = math.prod(out_shape)
    out = torch.empty(out_shape, device=q.device, dtype=out_dtype)
    if rows == 0:
        return out
    if cols == 0:
        return out.zero_()
    _hip.call(
        "fxpr_fixed_row_sum", q_c.data_ptr(), _hip.DTYPE_CODE[q_c.dtype], out.data_ptr(),
        int(int_bits), rows, cols, _hip.stream_ptr(q.device),
    )
    return out


def _as_2d(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1])


def _rms_launch(x, w, residual, eps):
    """Validation and copy-back rules of the reference's _common_launch
    (fxpr_vllm/_triton/rms_norm.py:78-134). The sum of squares has its own
    per-row block floating-point integer format (csrc/rows.hip), so, like the
    reference's launcher, this takes no fixed-point knobs."""
    if not x.is_cuda or not w.is_cuda:
        raise RuntimeError("rms_norm: x and w must be CUDA")
    if x.dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"rms_norm: unsupported input dtype {x.dtype}; expected one of {_SUPPORTED_DTYPES}")
    if w.dtype != x.dtype:
        raise TypeError("rms_norm: weight dtype must match input dtype")
    if residual is not None:
        if not residual.is_cuda:
            raise RuntimeError("rms_norm: residual must be CUDA")
        if residual.dtype != x.dtype:
            raise TypeError("rms_norm: residual dtype must match input dtype")
        if residual.shape != x.shape:
            raise ValueError("rms_norm: residual shape must match x")

    x_2d = _as_2d(x).contiguous()
    y_2d = torch.empty_like(x_2d)
    r_storage = None
    if residual is not None:
        r_2d = _as_2d(residual)
        r_storage = r_2d if r_2d.is_contiguous() else r_2d.contiguous()

    rows, hidden = x_2d.shape
    if rows == 0 or hidden == 0:
        if residual is not None and r_storage.data_ptr() != residual.data_ptr():
            residual.copy_(r_storage.view_as(residual))
        return y_2d.view_as(x)
    if w.numel() != hidden:
        raise ValueError(f"rms_norm: weight has {w.numel()} elements, hidden size is {hidden}")
    w_c = w.contiguous()

    _hip.call(
        "fxpr_rms_norm", x_2d.data_ptr(), _hip.ptr(r_storage), w_c.data_ptr(), y_2d.data_ptr(),
        _hip.DTYPE_CODE[x.dtype], rows, hidden, float(eps), _hip.stream_ptr(x.device),
    )
    if residual is not None and r_storage.data_ptr() != residual.data_ptr():
        residual.copy_(r_storage.view_as(residual))
    return y_2d.view_as(x)


def rms_norm_fxp_run(x, w, eps):
    """fxpr_vllm/_triton/rms_norm.py:137-142."""
    return _rms_launch(x, w, None, eps)


def rms_norm_fxp_residual_run(x, residual, w, eps):
    """fxpr_vllm/_triton/rms_norm.py:145-151 (mutates residual)."""
    return _rms_launch(x, w, residual, eps)


def log_softmax_fxp_run(x, int_bits, frac_bits, out_dtype=None):
    """Deterministic log-softmax over the last dim (fp32 / f16 / bf16 in;
    same dtype or fp32 out)."""
    if not x.is_cuda:
        raise RuntimeError("log_softmax_fxp: input must be CUDA")
    if x.dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"log_softmax_fxp: unsupported input dtype {x.dtype}; expected one of {_SUPPORTED_DTYPES}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in (x.dtype, torch.float32):
        raise TypeError(f"log_softmax_fxp: output dtype must be {x.dtype} or torch.float32, got {out_dtype}")
    b, f = _bits(int_bits, frac_bits)
    x_2d = _as_2d(x).contiguous() if x.dim() > 0 else x.reshape(1, 1)
    y_2d = torch.empty(x_2d.shape, device=x.device, dtype=out_dtype)
    rows, cols = x_2d.shape
    if rows and cols:
        _hip.call(
            "fxpr_log_softmax", x_2d.data_ptr(), _hip.DTYPE_CODE[x.dtype], y_2d.data_ptr(),
            _hip.DTYPE_CODE[out_dtype], rows, cols, b, f, _hip.stream_ptr(x.device),
        )
    return y_2d.view(x.shape)


# ---------------------------------------------------------------------------
# Vocab-parallel log-softmax: each shard holds some columns of every row.
# MAX of the shards' row maxima, then integer SUM of the shards' row sums
# against that maximum, then each shard's outputs (the exchanges a
# vocab-parallel lm_head needs between devices; csrc/rows.hip).


def _shard_rows(x: torch.Tensor, what: str) -> torch.Tensor:
    if not x.is_cuda:
        raise RuntimeError(f"{what}: input must be CUDA")
    if x.dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"{what}: unsupported input dtype {x.dtype}; expected one of {_SUPPORTED_DTYPES}")
    if x.dim() == 0:
        raise ValueError(f"{what}: input needs a column dimension")
    return _as_2d(x).contiguous()


def _row_stat(t: torch.Tensor, x: torch.Tensor, dtype: torch.dtype, what: str, name: str) -> torch.Tensor:
    if not t.is_cuda or t.dtype != dtype:
        raise TypeError(f"{what}: {name} must be a CUDA {dtype} tensor")
    if tuple(t.shape) != tuple(x.shape[:-1]):
        raise ValueError(f"{what}: {name} must have shape {tuple(x.shape[:-1])}")
    return t.contiguous()


def log_softmax_shard_max_run(x: torch.Tensor) -> torch.Tensor:
    """Row maxima (fp32) of this shard's columns."""
    x_2d = _shard_rows(x, "log_softmax_fxp_shard_max")
    out = torch.empty(x.shape[:-1], device=x.device, dtype=torch.float32)
    rows, cols = x_2d.shape
    if rows:
        _hip.call("fxpr_log_softmax_shard_max", x_2d.data_ptr(), _hip.DTYPE_CODE[x.dtype], out.data_ptr(), rows,
                  cols, _hip.stream_ptr(x.device))
    return out


def log_softmax_shard_sum_run(x: torch.Tensor, row_max: torch.Tensor, int_bits: int, frac_bits: int) -> torch.Tensor:
    """Exact int64 row sums of this shard's terms against the combined maxima."""
    what = "log_softmax_fxp_shard_sum"
    x_2d = _shard_rows(x, what)
    m = _row_stat(row_max, x, torch.float32, what, "row_max")
    b, f = _bits(int_bits, frac_bits)
    if f > 32:
        raise ValueError(f"{what}: frac_bits above 32 can overflow the int64 row sums")
    out = torch.empty(x.shape[:-1], device=x.device, dtype=torch.int64)
    rows, cols = x_2d.shape
    if rows:
        _hip.call("fxpr_log_softmax_shard_sum", x_2d.data_ptr(), _hip.DTYPE_CODE[x.dtype], m.data_ptr(),
                  out.data_ptr(), rows, cols, b, f, _hip.stream_ptr(x.device))
    return out


def log_softmax_shard_finish_run(x: torch.Tensor, row_max: torch.Tensor, row_sum: torch.Tensor, frac_bits: int,
                                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """This shard's log-probabilities from the combined maxima and sums."""
    what = "log_softmax_fxp_shard_finish"
    x_2d = _shard_rows(x, what)
    m = _row_stat(row_max, x, torch.float32, what, "row_max")
    s = _row_stat(row_sum, x, torch.int64, what, "row_sum")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in (x.dtype, torch.float32):
        raise TypeError(f"{what}: output dtype must be {x.dtype} or torch.float32, got {out_dtype}")
    y = torch.empty(x_2d.shape, device=x.device, dtype=out_dtype)
    rows, cols = x_2d.shape
    if rows and cols:
        _hip.call("fxpr_log_softmax_shard_finish", x_2d.data_ptr(), _hip.DTYPE_CODE[x.dtype], m.data_ptr(),
                  s.data_ptr(), y.data_ptr(), _hip.DTYPE_CODE[out_dtype], rows, cols, int(frac_bits),
                  _hip.stream_ptr(x.device))
    return y.view(x.shape)
