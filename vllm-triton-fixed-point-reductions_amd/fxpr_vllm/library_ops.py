"""Fake (meta) impls for torch.compile / Dynamo, plus torch.ops.fxpr aliases.

Output shapes and dtypes follow the reference fakes
(fxpr_vllm/library_ops.py:28-71); the build-only ops get their own.
"""

from __future__ import annotations

import torch

from . import _lib  # noqa: F401  (defines the schemas)


def _int_dtype_for_bits(int_bits: int) -> torch.dtype:
    if int_bits == 16:
        return torch.int16
    if int_bits == 32:
        return torch.int32
    if int_bits == 64:
        return torch.int64
    raise ValueError(f"int_bits must be 16/32/64, got {int_bits}")


def _float_dtype_for_bits(float_bits: int) -> torch.dtype:
    if float_bits == 16:
        return torch.float16
    if float_bits == 32:
        return torch.float32
    if float_bits == 64:
        return torch.float64
    raise ValueError(f"float_bits must be 16/32/64, got {float_bits}")


@torch.library.register_fake("fxpr::float_to_fixed")
def _float_to_fixed_fake(x, int_bits, fxp_frac_bits):
    return torch.empty_like(x, dtype=_int_dtype_for_bits(int(int_bits)))


@torch.library.register_fake("fxpr::fixed_to_float")
def _fixed_to_float_fake(x, float_bits, fxp_frac_bits):
    return torch.empty_like(x, dtype=_float_dtype_for_bits(int(float_bits)))


@torch.library.register_fake("fxpr::rms_norm_fxp")
def _rms_norm_fxp_fake(x, weight_fp32, eps):
    return torch.empty_like(x)


@torch.library.register_fake("fxpr::rms_norm_fxp_residual")
def _rms_norm_fxp_residual_fake(x, residual, weight_fp32, eps):
    return torch.empty_like(x)


@torch.library.register_fake("fxpr::gemm_fxp")
def _gemm_fxp_fake(a, b, bias, fxp_int_bits, fxp_frac_bits):
    return a.new_empty((a.shape[0], b.shape[1]))


@torch.library.register_fake("fxpr::unified_attention_fxp")
def _unified_attention_fxp_fake(q, kv_cache, o, query_start_loc, seq_lens, block_table,
                                max_query_len, alibi_slopes, is_causal, softmax_scale,
                                fxp_int_bits, fxp_frac_bits, logit_softcap, window_size,
                                num_kv_splits):
    return None


@torch.library.register_fake("fxpr::fixed_row_sum")
def _fixed_row_sum_fake(q, int_bits):
    shape = q.shape[:-1] if q.dim() else ()
    return q.new_empty(shape, dtype=_int_dtype_for_bits(int(int_bits)))


@torch.library.register_fake("fxpr::log_softmax_fxp")
def _log_softmax_fxp_fake(x, fxp_int_bits, fxp_frac_bits, out_dtype=None):
    return torch.empty_like(x, dtype=x.dtype if out_dtype is None else out_dtype)


@torch.library.register_fake("fxpr::sample_greedy_fxp")
def _sample_greedy_fxp_fake(logits, num_logprobs, fxp_int_bits, fxp_frac_bits):
    lead = tuple(logits.shape[:-1])
    k = int(num_logprobs)
    return (logits.new_empty(lead, dtype=torch.int64), logits.new_empty(lead, dtype=torch.float32),
            logits.new_empty(lead + (k,), dtype=torch.int64), logits.new_empty(lead + (k,), dtype=torch.float32))


@torch.library.register_fake("fxpr::reshape_and_cache")
def _reshape_and_cache_fake(key, value, kv_cache, slot_mapping):
    return None


@torch.library.register_fake("fxpr::gemm_fxp_partial")
def _gemm_fxp_partial_fake(a, b, fxp_int_bits, fxp_frac_bits):
    return a.new_empty((a.shape[0], b.shape[1]), dtype=torch.int64 if int(fxp_int_bits) == 64 else torch.int32)


@torch.library.register_fake("fxpr::gemm_fxp_finish")
def _gemm_fxp_finish_fake(acc, bias, fxp_int_bits, fxp_frac_bits, out_dtype):
    return acc.new_empty(acc.shape, dtype=out_dtype)


@torch.library.register_fake("fxpr::log_softmax_fxp_shard_max")
def _log_softmax_fxp_shard_max_fake(x):
    return x.new_empty(x.shape[:-1], dtype=torch.float32)


@torch.library.register_fake("fxpr::log_softmax_fxp_shard_sum")
def _log_softmax_fxp_shard_sum_fake(x, row_max, fxp_int_bits, fxp_frac_bits):
    return x.new_empty(x.shape[:-1], dtype=torch.int64)


@torch.library.register_fake("fxpr::log_softmax_fxp_shard_finish")
def _log_softmax_fxp_shard_finish_fake(x, row_max, row_sum, fxp_frac_bits, out_dtype=None):
    return torch.empty_like(x, dtype=x.dtype if out_dtype is None else out_dtype)


gemm_fxp = torch.ops.fxpr.gemm_fxp
gemm_fxp_partial = torch.ops.fxpr.gemm_fxp_partial
gemm_fxp_finish = torch.ops.fxpr.gemm_fxp_finish
log_softmax_fxp_shard_max = torch.ops.fxpr.log_softmax_fxp_shard_max
log_softmax_fxp_shard_sum = torch.ops.fxpr.log_softmax_fxp_shard_sum
log_softmax_fxp_shard_finish = torch.ops.fxpr.log_softmax_fxp_shard_finish
rms_norm_fxp = torch.ops.fxpr.rms_norm_fxp
rms_norm_fxp_residual = torch.ops.fxpr.rms_norm_fxp_residual
float_to_fixed = torch.ops.fxpr.float_to_fixed
fixed_to_float = torch.ops.fxpr.fixed_to_float
fixed_row_sum = torch.ops.fxpr.fixed_row_sum
log_softmax_fxp = torch.ops.fxpr.log_softmax_fxp
reshape_and_cache = torch.ops.fxpr.reshape_and_cache
sample_greedy_fxp = torch.ops.fxpr.sample_greedy_fxp
unified_attention_fxp = torch.ops.fxpr.unified_attention_fxp
