"""Fixed-point GEMM launcher (csrc/gemm.hip).

Host half of the reference's gemm_fxp_run (fxpr_vllm/_triton/gemm.py:612-763):
allocate C with the caching allocator, pick the split count (a static policy
in the library replaces Triton autotuning and warm-up split timing, since no
choice ever changes the bits), hand raw pointers and strides to fxpr_gemm.
"""

from __future__ import annotations

import torch

from .. import _hip
from .fxp import fxp_constants

# K-tile width per input dtype: the determinism unit (one fp32 MFMA partial is
# quantised per tile). Same values as the reference's _BLOCK_K_BY_DTYPE
# (fxpr_vllm/_triton/gemm.py:26-30).
_BLOCK_K_BY_DTYPE = {
    torch.float16: 128,
    torch.bfloat16: 128,
    torch.float32: 64,
}
_SUPPORTED_DTYPES = tuple(_BLOCK_K_BY_DTYPE)


def resolve_split_k(M: int, N: int, K: int, dtype: torch.dtype, int_bits: int = 32, split_k: int = 0) -> int:
    """Split count the library will use for int_bits-bit sums (split_k 0 = its
    automatic policy)."""
    return _hip.load().fxpr_gemm_splits(M, N, K, _hip.DTYPE_CODE[dtype], int(int_bits), int(split_k))


def gemm_fxp_run(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None, int_bits: int,
                 fxp_frac_bits: int, split_k: int = 0) -> torch.Tensor:
    if not (a.is_cuda and b.is_cuda):
        raise RuntimeError("gemm_fxp: a and b must be CUDA")
    if a.dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"gemm_fxp: unsupported dtype {a.dtype}; expected one of {_SUPPORTED_DTYPES}")
    if b.dtype != a.dtype:
        raise TypeError("gemm_fxp: a and b must share a dtype")
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"gemm_fxp: shape mismatch {tuple(a.shape)} x {tuple(b.shape)}")
    fxp_constants(int(int_bits), int(fxp_frac_bits))

    M, K = a.shape
    N = b.shape[1]
    c = torch.empty((M, N), device=a.device, dtype=a.dtype)
    if M == 0 or N == 0:
        return c
    if a.stride(1) != 1 and K > 1:
        a = a.contiguous()
    if b.stride(0) != 1 and b.stride(1) != 1:
        b = b.contiguous()
    bias_f32 = None
    if bias is not None:
        if bias.numel() != N:
            raise ValueError(f"gemm_fxp: bias has {bias.numel()} elements, expected {N}")
        bias_f32 = bias.reshape(N).to(torch.float32).contiguous()

    lib = _hip.load()
    code = _hip.DTYPE_CODE[a.dtype]
    ws_bytes = lib.fxpr_gemm_workspace_bytes(M, N, K, code, int(int_bits), int(split_k))
    ws = torch.empty(ws_bytes, device=a.device, dtype=torch.uint8) if ws_bytes > 0 else None
    _hip.call(
        "fxpr_gemm", a.data_ptr(), b.data_ptr(), _hip.ptr(bias_f32), c.data_ptr(), code,
        M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1),
        int(int_bits), int(fxp_frac_bits), int(split_k), _hip.ptr(ws), ws_bytes,
        _hip.stream_ptr(a.device),
    )
    return c


# ---------------------------------------------------------------------------
# Row-parallel shards (K split over devices): each shard's integer
# accumulators, summed across shards with integer adds (an all-reduce SUM on
# int32 / int64, whose order cannot change the bits), then one epilogue. No
# counterpart in the reference, whose row-parallel linears all-reduce bf16
# outputs (fxpr_vllm/quantisation_config.py:80-96 sets the layers up).


def acc_dtype_for_bits(int_bits: int) -> torch.dtype:
    """The accumulator type of the partial sums: int32 for 16- and 32-bit
    formats (a 16-bit format wraps at the epilogue), int64 for 64-bit."""
    return torch.int64 if int(int_bits) == 64 else torch.int32


def gemm_fxp_partial_run(a: torch.Tensor, b: torch.Tensor, int_bits: int, fxp_frac_bits: int) -> torch.Tensor:
    """acc[m, n] = sum over this call's K-tiles of RNE_sat(P_t[m, n] * 2^f),
    wrapping. A K-shard's partials add up to the unsharded GEMM's accumulator
    when its first column is a K-tile boundary of the full K (a multiple of
    128 for 16-bit inputs, 64 for fp32)."""
    if not (a.is_cuda and b.is_cuda):
        raise RuntimeError("gemm_fxp_partial: a and b must be CUDA")
    if a.dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"gemm_fxp_partial: unsupported dtype {a.dtype}; expected one of {_SUPPORTED_DTYPES}")
    if b.dtype != a.dtype:
        raise TypeError("gemm_fxp_partial: a and b must share a dtype")
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"gemm_fxp_partial: shape mismatch {tuple(a.shape)} x {tuple(b.shape)}")
    fxp_constants(int(int_bits), int(fxp_frac_bits))
    M, K = a.shape
    N = b.shape[1]
    acc = torch.empty((M, N), device=a.device, dtype=acc_dtype_for_bits(int_bits))
    if M == 0 or N == 0:
        return acc
    if a.stride(1) != 1 and K > 1:
        a = a.contiguous()
    if b.stride(0) != 1 and b.stride(1) != 1:
        b = b.contiguous()
    _hip.call(
        "fxpr_gemm_partial", a.data_ptr(), b.data_ptr(), acc.data_ptr(), _hip.DTYPE_CODE[a.dtype],
        M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), int(int_bits), int(fxp_frac_bits),
        _hip.stream_ptr(a.device),
    )
    return acc


def gemm_fxp_finish_run(acc: torch.Tensor, bias: torch.Tensor | None, int_bits: int, fxp_frac_bits: int,
                        out_dtype: torch.dtype) -> torch.Tensor:
    """C = IO(fl32(acc wrapped to int_bits) * 2^-f (+ bias)): gemm_fxp's
    epilogue on summed shard accumulators."""
    if not acc.is_cuda:
        raise RuntimeError("gemm_fxp_finish: acc must be CUDA")
    if acc.dtype != acc_dtype_for_bits(int_bits):
        raise TypeError(f"gemm_fxp_finish: acc must be {acc_dtype_for_bits(int_bits)} for {int_bits}-bit sums")
    if out_dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"gemm_fxp_finish: unsupported out_dtype {out_dtype}; expected one of {_SUPPORTED_DTYPES}")
    if acc.dim() != 2:
        raise ValueError("gemm_fxp_finish: acc must be [M, N]")
    fxp_constants(int(int_bits), int(fxp_frac_bits))
    M, N = acc.shape
    c = torch.empty((M, N), device=acc.device, dtype=out_dtype)
    if M == 0 or N == 0:
        return c
    acc = acc.contiguous()
    bias_f32 = None
    if bias is not None:
        if bias.numel() != N:
            raise ValueError(f"gemm_fxp_finish: bias has {bias.numel()} elements, expected {N}")
        bias_f32 = bias.reshape(N).to(torch.float32).contiguous()
    _hip.call(
        "fxpr_gemm_finish", acc.data_ptr(), _hip.ptr(bias_f32), c.data_ptr(), _hip.DTYPE_CODE[out_dtype], M, N,
        c.stride(0), c.stride(1), int(int_bits), int(fxp_frac_bits), _hip.stream_ptr(acc.device),
    )
    return c
