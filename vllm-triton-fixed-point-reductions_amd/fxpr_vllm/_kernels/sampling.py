"""Greedy sampling launcher (csrc/sampling.hip).

No counterpart in the reference, which lists fxpr_vllm/sampling.py
(README.md:69) without shipping it: the step after the lm_head GEMM.
"""

from __future__ import annotations

import torch

from .. import _hip
from .fxp import fxp_constants

MAX_LOGPROBS = 64
_SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def sample_greedy_fxp_run(logits: torch.Tensor, num_logprobs: int, int_bits: int, frac_bits: int):
    """(token ids int64 [R], their log-probs fp32 [R], top-k ids int64 [R, k],
    top-k log-probs fp32 [R, k]) for logits [..., V] flattened to R rows."""
    if not logits.is_cuda:
        raise RuntimeError("sample_greedy_fxp: logits must be CUDA")
    if logits.dtype not in _SUPPORTED_DTYPES:
        raise TypeError(f"sample_greedy_fxp: unsupported dtype {logits.dtype}; expected one of "
                        f"{_SUPPORTED_DTYPES}")
    if logits.dim() == 0:
        raise ValueError("sample_greedy_fxp: logits need a vocabulary dimension")
    fxp_constants(int(int_bits), int(frac_bits))
    k = int(num_logprobs)
    vocab = logits.shape[-1]
    if vocab == 0:
        raise ValueError("sample_greedy_fxp: empty vocabulary")
    if not 0 <= k <= min(MAX_LOGPROBS, vocab):
        raise ValueError(f"sample_greedy_fxp: num_logprobs must be in [0, {min(MAX_LOGPROBS, vocab)}], got {k}")
    x = logits.reshape(-1, vocab).contiguous()
    rows = x.shape[0]
    dev = logits.device
    ids = torch.empty(rows, device=dev, dtype=torch.int64)
    lp = torch.empty(rows, device=dev, dtype=torch.float32)
    topk_ids = torch.empty(rows, k, device=dev, dtype=torch.int64)
    topk_lp = torch.empty(rows, k, device=dev, dtype=torch.float32)
    if rows:
        # few rows: the library spreads each row over several workgroups, its
        # partials in this workspace (caching allocator: capture-safe)
        ws_bytes = _hip.load().fxpr_sample_greedy_workspace_bytes(rows, k)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes > 0 else None
        _hip.call("fxpr_sample_greedy", x.data_ptr(), _hip.DTYPE_CODE[x.dtype], rows, vocab, k, int(int_bits),
                  int(frac_bits), ids.data_ptr(), lp.data_ptr(), _hip.ptr(topk_ids) if k else None,
                  _hip.ptr(topk_lp) if k else None, _hip.ptr(ws), ws_bytes, _hip.stream_ptr(dev))
    lead = tuple(logits.shape[:-1])
    return ids.view(lead), lp.view(lead), topk_ids.view(lead + (k,)), topk_lp.view(lead + (k,))
