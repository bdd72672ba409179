"""Paged KV-cache write launcher (csrc/cache.hip).

The step before attention in the backend's forward: key / value rows of the
step's tokens are scattered into the [num_blocks, 2, block_size,
num_kv_heads, head_size] cache at slot_mapping (block * block_size + offset;
negative = padding, skipped). Stands in for vLLM's reshape_and_cache_flash as
the reference backend calls it (fxpr_vllm/attention_backend.py:253-277).
"""

from __future__ import annotations

import torch

from .. import _hip

_SUPPORTED = (torch.float16, torch.bfloat16, torch.float32)


def reshape_and_cache_run(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                          slot_mapping: torch.Tensor) -> None:
    if not (key.is_cuda and value.is_cuda and kv_cache.is_cuda and slot_mapping.is_cuda):
        raise RuntimeError("reshape_and_cache: tensors must be CUDA")
    if kv_cache.dim() != 5 or kv_cache.shape[1] != 2:
        raise ValueError("kv_cache must be (num_blocks, 2, block_size, num_kv_heads, head_size)")
    if kv_cache.dtype not in _SUPPORTED:
        raise TypeError(f"reshape_and_cache: unsupported cache dtype {kv_cache.dtype}")
    if key.dtype != kv_cache.dtype or value.dtype != kv_cache.dtype:
        raise TypeError("key, value and kv_cache must share a dtype")
    num_blocks, _, block_size, num_kv_heads, head_size = kv_cache.shape
    if key.dim() == 2:
        key = key.view(key.shape[0], num_kv_heads, head_size)
    if value.dim() == 2:
        value = value.view(value.shape[0], num_kv_heads, head_size)
    if key.shape != value.shape or tuple(key.shape[1:]) != (num_kv_heads, head_size):
        raise ValueError("key / value must be [num_tokens, num_kv_heads, head_size] matching the cache")
    num_tokens = key.shape[0]
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] < num_tokens:
        raise ValueError("slot_mapping must be 1-D with one slot per token")
    if num_tokens == 0:
        return
    if key.stride(2) != 1:
        key = key.contiguous()
    if value.stride(2) != 1:
        value = value.contiguous()
    slots = slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.to(torch.int64)
    slots = slots.contiguous()
    k_cache = kv_cache.select(1, 0)
    v_cache = kv_cache.select(1, 1)
    if k_cache.stride(3) != 1:
        raise ValueError("kv_cache must be contiguous along head_size")
    _hip.call(
        "fxpr_reshape_and_cache",
        key.data_ptr(), value.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        _hip.DTYPE_CODE[kv_cache.dtype], slots.data_ptr(), num_tokens, num_kv_heads, head_size,
        block_size, num_blocks, key.stride(0), key.stride(1), value.stride(0), value.stride(1),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2),
        _hip.stream_ptr(key.device),
    )
