"""DeterministicRMSNorm: vLLM's RMSNorm running the fixed-point kernels.

Counterpart of the reference class (fxpr_vllm/rms_norm.py:9-27): every
forward variant vLLM may dispatch to is bound to the fixed-point path, so the
layer never falls back to a batch-variant kernel. On ROCm vLLM's CustomOp
dispatches to ``forward_hip`` (where RMSNorm may route to its own fused ROCm
kernels), so that entry is bound too, besides ``forward_cuda`` and
``forward_native`` (the torch.compile path).

Without vLLM the class derives from a minimal module with the attributes the
forward uses (``weight``, ``variance_epsilon``), so the layer can be built
and tested on its own; the arithmetic is the same HIP kernels either way.
"""

from __future__ import annotations

import torch

from .library_ops import rms_norm_fxp, rms_norm_fxp_residual


class _StandaloneRMSNorm(torch.nn.Module):
    """The parts of vLLM's RMSNorm the fixed-point forward relies on."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, dtype: torch.dtype | None = None,
                 **_unused) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.variance_epsilon = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden_size, dtype=dtype), requires_grad=False)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        return self.forward_cuda(x, residual)


def _rms_norm_base() -> type:
    try:
        from vllm.model_executor.layers.layernorm import RMSNorm
    except ImportError:
        return _StandaloneRMSNorm
    return RMSNorm


class DeterministicRMSNorm(_rms_norm_base()):
    def _forward_fxp(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        # fused residual: residual <- x + residual (in place), returns (normed, residual)
        if residual is not None:
            out = rms_norm_fxp_residual(x, residual, self.weight, self.variance_epsilon)
            return out, residual
        return rms_norm_fxp(x, self.weight, self.variance_epsilon)

    forward_cuda = _forward_fxp
    forward_hip = _forward_fxp
    forward_native = _forward_fxp
