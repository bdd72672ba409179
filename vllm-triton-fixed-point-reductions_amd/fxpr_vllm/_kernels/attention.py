"""Unified paged attention launcher (csrc/attn*.hip).

Host half of the reference's unified_attention_fxp_run
(fxpr_vllm/_triton/attention.py:692-953): same validation order, error
classes and split policy inputs (host-side shapes only, no device sync, so it
is safe under graph capture); the kernels themselves are in the HIP library.
"""

from __future__ import annotations

import math

import torch

from .. import _hip
from .fxp import fxp_constants

_RCP_LN2 = 1.4426950408889634
_SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)

# Key-tile width per dtype: the determinism unit of the weighted-V partials
# (reference _BLOCK_N_BY_DTYPE, attention.py:32-36). Tiles are aligned to
# absolute key positions.
_BLOCK_N_BY_DTYPE = {torch.float16: 64, torch.bfloat16: 64, torch.float32: 32}


def pick_num_splits(num_kv_splits: int, num_requests: int, num_kv_heads: int, group: int,
                    max_query_len: int, max_blocks: int, page_size: int) -> int:
    return _hip.load().fxpr_attention_splits(num_requests, num_kv_heads, group, max_query_len,
                                             max_blocks, page_size, int(num_kv_splits))


def unified_attention_fxp_run(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    o: torch.Tensor,
    query_start_loc: torch.Tensor,
    seq_lens: torch.Tensor,
    block_table: torch.Tensor,
    max_query_len: int,
    alibi_slopes: torch.Tensor | None,
    is_causal: bool,
    softmax_scale: float | None,
    fxp_int_bits: int,
    fxp_frac_bits: int,
    logit_softcap: float,
    window_size: int,
    num_kv_splits: int,
    static_scratch: bool = False,
) -> None:
    """static_scratch=True calls fxpr_unified_attention_noalloc: no workspace
    is allocated (the split partials live in the library's static device
    array; a launch needing more raises RuntimeError)."""
    if not (q.is_cuda and kv_cache.is_cuda and o.is_cuda):
        raise RuntimeError("unified_attention_fxp: tensors must be CUDA")
    if q.dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"unified_attention_fxp: unsupported q dtype {q.dtype}")
    if kv_cache.dim() != 5 or kv_cache.shape[1] != 2:
        raise ValueError("kv_cache must be (num_blocks, 2, page_size, num_kv_heads, head_dim)")
    if kv_cache.dtype != q.dtype or o.dtype != q.dtype:
        raise TypeError("kv_cache and o must share dtype with q")
    if query_start_loc.dtype != torch.int32:
        raise TypeError("query_start_loc must be int32")
    if seq_lens.dtype != torch.int32:
        raise TypeError("seq_lens must be int32")
    if block_table.dtype != torch.int32:
        raise TypeError("block_table must be int32")
    if num_kv_splits < 0:
        raise ValueError(f"num_kv_splits must be >= 0, got {num_kv_splits}")
    has_alibi = alibi_slopes is not None and alibi_slopes.numel() > 0
    if has_alibi and alibi_slopes.dtype != torch.float32:
        raise TypeError("alibi_slopes must be float32")
    fxp_constants(int(fxp_int_bits), int(fxp_frac_bits))

    k_cache = kv_cache.select(1, 0)
    v_cache = kv_cache.select(1, 1)
    num_tokens, num_heads, head_dim = q.shape
    num_blocks, page_size, num_kv_heads = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    num_requests = seq_lens.shape[0]
    if num_heads % num_kv_heads != 0:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if k_cache.shape[3] != head_dim or o.shape != q.shape:
        raise ValueError("q, o and kv_cache head sizes must agree")
    if num_requests == 0 or num_tokens == 0:
        return
    if q.stride(2) != 1:
        q = q.contiguous()
    if k_cache.stride(3) != 1:
        raise ValueError("kv_cache must be contiguous along head_dim")
    out = o if o.stride(2) == 1 else torch.empty_like(o, memory_format=torch.contiguous_format)
    bt = block_table if block_table.dim() == 2 else block_table.reshape(num_requests, -1)
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    qsl = query_start_loc.contiguous()
    sl = seq_lens.contiguous()
    alibi = alibi_slopes.contiguous() if has_alibi else None

    ss = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(head_dim)
    ss_log2 = float(ss) * _RCP_LN2
    softcap_log2 = float(logit_softcap) * _RCP_LN2 if float(logit_softcap) > 0.0 else 0.0
    max_blocks = bt.shape[1]
    common = (
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), _hip.DTYPE_CODE[q.dtype],
        qsl.data_ptr(), sl.data_ptr(), bt.data_ptr(), _hip.ptr(alibi),
        num_requests, num_tokens, num_heads, num_kv_heads, head_dim, page_size,
        int(max_query_len), max_blocks, num_blocks,
        q.stride(0), q.stride(1), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2), out.stride(0), out.stride(1),
        bt.stride(0), int(bool(is_causal)), ss_log2, softcap_log2, max(0, int(window_size)),
        int(fxp_int_bits), int(fxp_frac_bits), int(num_kv_splits),
    )
    if static_scratch:
        _hip.call("fxpr_unified_attention_noalloc", *common, _hip.stream_ptr(q.device))
    else:
        ws_bytes = _hip.load().fxpr_attention_workspace_bytes(
            num_requests, num_tokens, num_heads, num_kv_heads, head_dim, int(fxp_int_bits),
            int(num_kv_splits), int(max_query_len), max_blocks, page_size)
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes > 0 else None
        _hip.call("fxpr_unified_attention", *common, _hip.ptr(ws), ws_bytes, _hip.stream_ptr(q.device))
    if out is not o:
        o.copy_(out)
