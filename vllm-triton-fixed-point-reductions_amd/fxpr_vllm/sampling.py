"""Deterministic greedy sampler with log-probabilities: the step after the lm_head.

The reference lists fxpr_vllm/sampling.py (README.md:69 of
Gursukh/vLLM-Triton-Fixed-Point-Reductions) without shipping it; this is the
build's own. It covers greedy decoding, the case whose tokens the fixed-point
GEMM, attention and RMSNorm make independent of batch composition:

  * the token of a row is the largest logit, ties to the lowest index, a NaN
    logit ranking above every number (torch.argmax's choice on the same row);
  * its log-probability, and optionally the top-k log-probabilities in the
    same order, are log_softmax_fxp's fp32 values bit for bit (one kernel,
    torch.ops.fxpr.sample_greedy_fxp, computes both from one pass over the
    logits);
  * the fixed-point format is FXPR_INT_BITS / FXPR_FRAC_BITS, as for the
    other ops.

Does not import vLLM.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import library_ops  # noqa: F401  (registers torch.ops.fxpr.*)
from ._kernels.sampling import MAX_LOGPROBS
from .config import get_runtime_config


@dataclass(frozen=True)
class GreedySample:
    token_ids: torch.Tensor        # [..., ] int64
    logprobs: torch.Tensor         # [..., ] fp32, log-probability of token_ids
    topk_token_ids: torch.Tensor   # [..., k] int64, largest logits first
    topk_logprobs: torch.Tensor    # [..., k] fp32


class DeterministicSampler(torch.nn.Module):
    """Greedy tokens and log-probabilities from logits [..., vocab]."""

    max_logprobs = MAX_LOGPROBS

    def forward(self, logits: torch.Tensor, num_logprobs: int = 0) -> GreedySample:
        cfg = get_runtime_config()
        ids, lp, topk_ids, topk_lp = torch.ops.fxpr.sample_greedy_fxp(logits, int(num_logprobs),
                                                                       cfg.fxp_int_bits, cfg.fxp_frac_bits)
        return GreedySample(ids, lp, topk_ids, topk_lp)

    @staticmethod
    def compute_logprobs(logits: torch.Tensor) -> torch.Tensor:
        """Full fp32 log-probabilities (the values forward() reports)."""
        cfg = get_runtime_config()
        return torch.ops.fxpr.log_softmax_fxp(logits, cfg.fxp_int_bits, cfg.fxp_frac_bits, torch.float32)
