"""torch.ops.fxpr.* schemas and their "CUDA"-key impls (HIP kernels).

The six reference schemas are kept verbatim (fxpr_vllm/_lib.py:13-33 of the
reference) so callers and torch.compile graphs are a drop-in; PyTorch-ROCm
dispatches HIP tensors through the CUDA key. Nine schemas are new in this
build: the shard halves of gemm_fxp and log_softmax_fxp for more than one
device (below), fixed_row_sum (the integer sum the reference's tests do with torch,
_tests/test_sum.py:12-16), log_softmax_fxp (listed in the reference
README.md:60 but not shipped), sample_greedy_fxp (the sampler of the
reference's README.md:69, likewise not shipped) and reshape_and_cache (the
KV-cache write the reference backend takes from vLLM,
attention_backend.py:253-277). Validation and error classes follow the
reference impls (_lib.py:36-129).
"""

from __future__ import annotations

import torch

from ._kernels import attention as _attention
from ._kernels import cache as _cache
from ._kernels import casts as _casts
from ._kernels import gemm as _gemm
from ._kernels import rows as _rows
from ._kernels import sampling as _sampling

_lib = torch.library.Library("fxpr", "DEF")

_lib.define("float_to_fixed(Tensor x, int int_bits, int fxp_frac_bits) -> Tensor")
_lib.define("fixed_to_float(Tensor x, int float_bits, int fxp_frac_bits) -> Tensor")
# RMSNorm's integer sum of squares has a per-row format of its own (no knobs).
_lib.define("rms_norm_fxp(Tensor x, Tensor weight_fp32, float eps) -> Tensor")
_lib.define(
    "rms_norm_fxp_residual(Tensor x, Tensor(a!) residual, Tensor weight_fp32, "
    "float eps) -> Tensor"
)
_lib.define(
    "gemm_fxp(Tensor a, Tensor b, Tensor? bias, int fxp_int_bits, "
    "int fxp_frac_bits) -> Tensor"
)
_lib.define(
    "unified_attention_fxp(Tensor q, Tensor kv_cache, Tensor(a!) o, "
    "Tensor query_start_loc, Tensor seq_lens, Tensor block_table, "
    "int max_query_len, Tensor? alibi_slopes, bool is_causal, "
    "float? softmax_scale, int fxp_int_bits, int fxp_frac_bits, "
    "float logit_softcap, int window_size, int num_kv_splits) -> ()"
)
_lib.define("fixed_row_sum(Tensor q, int int_bits) -> Tensor")
_lib.define(
    "log_softmax_fxp(Tensor x, int fxp_int_bits, int fxp_frac_bits, "
    "ScalarType? out_dtype=None) -> Tensor"
)
_lib.define(
    "reshape_and_cache(Tensor key, Tensor value, Tensor(a!) kv_cache, "
    "Tensor slot_mapping) -> ()"
)
_lib.define(
    "sample_greedy_fxp(Tensor logits, int num_logprobs, int fxp_int_bits, "
    "int fxp_frac_bits) -> (Tensor, Tensor, Tensor, Tensor)"
)
# Shard halves for more than one device: a K-sharded (row-parallel) GEMM's
# integer accumulators and their epilogue; a vocab-sharded log-softmax's row
# maxima, exact row sums and outputs. Summing / maxing the shard results
# across devices (integer all-reduces) gives the unsharded bits.
_lib.define("gemm_fxp_partial(Tensor a, Tensor b, int fxp_int_bits, int fxp_frac_bits) -> Tensor")
_lib.define(
    "gemm_fxp_finish(Tensor acc, Tensor? bias, int fxp_int_bits, int fxp_frac_bits, "
    "ScalarType out_dtype) -> Tensor"
)
_lib.define("log_softmax_fxp_shard_max(Tensor x) -> Tensor")
_lib.define(
    "log_softmax_fxp_shard_sum(Tensor x, Tensor row_max, int fxp_int_bits, int fxp_frac_bits) -> Tensor"
)
_lib.define(
    "log_softmax_fxp_shard_finish(Tensor x, Tensor row_max, Tensor row_sum, int fxp_frac_bits, "
    "ScalarType? out_dtype=None) -> Tensor"
)


def _check_frac_bits(n: int) -> None:
    if int(n) not in (8, 16, 32):
        raise ValueError(f"fxp_frac_bits must be 8/16/32, got {n}")


def _check_int_bits(n: int) -> None:
    if int(n) not in (16, 32, 64):
        raise ValueError(f"int_bits must be 16/32/64, got {n}")


def _float_to_fixed_cuda(x: torch.Tensor, int_bits: int, fxp_frac_bits: int):
    _check_int_bits(int_bits)
    _check_frac_bits(fxp_frac_bits)
    return _casts.float_to_fixed_run(x, int(int_bits), int(fxp_frac_bits))


def _fixed_to_float_cuda(x: torch.Tensor, float_bits: int, fxp_frac_bits: int):
    if int(float_bits) not in (16, 32, 64):
        raise ValueError(f"float_bits must be 16/32/64, got {float_bits}")
    _check_frac_bits(fxp_frac_bits)
    return _casts.fixed_to_float_run(x, int(float_bits), int(fxp_frac_bits))


def _rms_norm_fxp_cuda(x: torch.Tensor, weight: torch.Tensor, eps: float):
    return _rows.rms_norm_fxp_run(x, weight, float(eps))


def _rms_norm_fxp_residual_cuda(x: torch.Tensor, residual: torch.Tensor,
                                weight: torch.Tensor, eps: float):
    return _rows.rms_norm_fxp_residual_run(x, residual, weight, float(eps))


def _gemm_fxp_cuda(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None,
                   fxp_int_bits: int, fxp_frac_bits: int):
    _check_int_bits(fxp_int_bits)
    _check_frac_bits(fxp_frac_bits)
    return _gemm.gemm_fxp_run(a, b, bias, int(fxp_int_bits), int(fxp_frac_bits))


def _unified_attention_fxp_cuda(q, kv_cache, o, query_start_loc, seq_lens, block_table,
                                max_query_len, alibi_slopes, is_causal, softmax_scale,
                                fxp_int_bits, fxp_frac_bits, logit_softcap, window_size,
                                num_kv_splits):
    _check_int_bits(fxp_int_bits)
    _check_frac_bits(fxp_frac_bits)
    _attention.unified_attention_fxp_run(
        q, kv_cache, o, query_start_loc, seq_lens, block_table, int(max_query_len),
        alibi_slopes, bool(is_causal), None if softmax_scale is None else float(softmax_scale),
        int(fxp_int_bits), int(fxp_frac_bits), float(logit_softcap), int(window_size),
        int(num_kv_splits),
    )


def _fixed_row_sum_cuda(q: torch.Tensor, int_bits: int):
    _check_int_bits(int_bits)
    return _rows.fixed_row_sum_run(q, int(int_bits))


def _log_softmax_fxp_cuda(x: torch.Tensor, fxp_int_bits: int, fxp_frac_bits: int,
                          out_dtype: torch.dtype | None = None):
    _check_int_bits(fxp_int_bits)
    _check_frac_bits(fxp_frac_bits)
    return _rows.log_softmax_fxp_run(x, int(fxp_int_bits), int(fxp_frac_bits), out_dtype)


def _reshape_and_cache_cuda(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                            slot_mapping: torch.Tensor):
    _cache.reshape_and_cache_run(key, value, kv_cache, slot_mapping)


def _sample_greedy_fxp_cuda(logits: torch.Tensor, num_logprobs: int, fxp_int_bits: int,
                            fxp_frac_bits: int):
    _check_int_bits(fxp_int_bits)
    _check_frac_bits(fxp_frac_bits)
    return _sampling.sample_greedy_fxp_run(logits, int(num_logprobs), int(fxp_int_bits), int(fxp_frac_bits))


def _gemm_fxp_partial_cuda(a, b, fxp_int_bits, fxp_frac_bits):
    _check_int_bits(fxp_int_bits)
    _check_frac_bits(fxp_frac_bits)
    return _gemm.gemm_fxp_partial_run(a, b, int(fxp_int_bits), int(fxp_frac_bits))


def _gemm_fxp_finish_cuda(acc, bias, fxp_int_bits, fxp_frac_bits, out_dtype):
    _check_int_bits(fxp_int_bits)
    _check_frac_bits(fxp_frac_bits)
    return _gemm.gemm_fxp_finish_run(acc, bias, int(fxp_int_bits), int(fxp_frac_bits), out_dtype)


def _log_softmax_fxp_shard_max_cuda(x):
    return _rows.log_softmax_shard_max_run(x)


def _log_softmax_fxp_shard_sum_cuda(x, row_max, fxp_int_bits, fxp_frac_bits):
    _check_int_bits(fxp_int_bits)
    _check_frac_bits(fxp_frac_bits)
    return _rows.log_softmax_shard_sum_run(x, row_max, int(fxp_int_bits), int(fxp_frac_bits))


def _log_softmax_fxp_shard_finish_cuda(x, row_max, row_sum, fxp_frac_bits, out_dtype=None):
    _check_frac_bits(fxp_frac_bits)
    return _rows.log_softmax_shard_finish_run(x, row_max, row_sum, int(fxp_frac_bits), out_dtype)


# Register after definition so the functions stay importable by name.
_lib.impl("float_to_fixed", _float_to_fixed_cuda, "CUDA")
_lib.impl("fixed_to_float", _fixed_to_float_cuda, "CUDA")
_lib.impl("rms_norm_fxp", _rms_norm_fxp_cuda, "CUDA")
_lib.impl("rms_norm_fxp_residual", _rms_norm_fxp_residual_cuda, "CUDA")
_lib.impl("gemm_fxp", _gemm_fxp_cuda, "CUDA")
_lib.impl("unified_attention_fxp", _unified_attention_fxp_cuda, "CUDA")
_lib.impl("fixed_row_sum", _fixed_row_sum_cuda, "CUDA")
_lib.impl("log_softmax_fxp", _log_softmax_fxp_cuda, "CUDA")
_lib.impl("reshape_and_cache", _reshape_and_cache_cuda, "CUDA")
_lib.impl("sample_greedy_fxp", _sample_greedy_fxp_cuda, "CUDA")
_lib.impl("gemm_fxp_partial", _gemm_fxp_partial_cuda, "CUDA")
_lib.impl("gemm_fxp_finish", _gemm_fxp_finish_cuda, "CUDA")
_lib.impl("log_softmax_fxp_shard_max", _log_softmax_fxp_shard_max_cuda, "CUDA")
_lib.impl("log_softmax_fxp_shard_sum", _log_softmax_fxp_shard_sum_cuda, "CUDA")
_lib.impl("log_softmax_fxp_shard_finish", _log_softmax_fxp_shard_finish_cuda, "CUDA")
