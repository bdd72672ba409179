"""Hook the fixed-point layers into vLLM (called from register()).

Same two patches as the reference (fxpr_vllm/monkey_patches.py:12-43):

* patch_rms_norm: the custom-op registries and the layernorm module's
  RMSNorm name point at DeterministicRMSNorm, so models built afterwards get
  it. Model modules imported before the patch keep the class they bound at
  import; that case is logged.
* patch_attention_backend: registers DeterministicAttentionBackend as
  AttentionBackendEnum.CUSTOM (select it with attention_backend="CUSTOM").
"""

from __future__ import annotations

import logging
import sys

logger = logging.getLogger("fxpr_vllm")


def patch_rms_norm() -> None:
    import vllm.model_executor.layers.layernorm as layernorm_mod
    from vllm.model_executor.custom_op import op_registry, op_registry_oot

    from .rms_norm import DeterministicRMSNorm

    DeterministicRMSNorm.name = "rms_norm"
    op_registry["rms_norm"] = DeterministicRMSNorm
    op_registry_oot["RMSNorm"] = DeterministicRMSNorm
    layernorm_mod.RMSNorm = DeterministicRMSNorm
    early = [m for m in sys.modules if m.startswith("vllm.model_executor.models.")]
    if early:
        logger.warning("patched RMSNorm, but %d model module(s) were imported earlier and keep "
                       "the original class", len(early))


def patch_attention_backend() -> None:
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    from .attention_backend import DeterministicAttentionBackend

    path = f"{DeterministicAttentionBackend.__module__}.{DeterministicAttentionBackend.__qualname__}"
    register_backend(AttentionBackendEnum.CUSTOM, class_path=path)
