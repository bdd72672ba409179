"""Points vLLM at the fixed-point layers. Called by register().

Two hooks, the same two the reference installs (fxpr_vllm/monkey_patches.py:
12-43 of Gursukh/vLLM-Triton-Fixed-Point-Reductions):

* install_rms_norm() makes DeterministicRMSNorm the class vLLM builds for
  "rms_norm". vLLM resolves the class through three names: its in-tree
  custom-op registry ("rms_norm"), its out-of-tree registry ("RMSNorm") and
  the `RMSNorm` attribute of vllm.model_executor.layers.layernorm. A model
  module that ran `from ...layernorm import RMSNorm` before the hook keeps the
  class it bound; the hook names those modules in a warning.
* install_attention_backend() registers DeterministicAttentionBackend as
  AttentionBackendEnum.CUSTOM (selected with attention_backend="CUSTOM").
  The backend is registered by dotted path, so its module (and vLLM's
  attention metadata classes) load only when vLLM selects it.

patch_rms_norm / patch_attention_backend are the reference's names for the
two hooks.
"""

from __future__ import annotations

import logging
import sys

logger = logging.getLogger("fxpr_vllm")

BACKEND_CLASS_PATH = "fxpr_vllm.attention_backend.DeterministicAttentionBackend"
RMS_NORM_OP_NAME = "rms_norm"


def _modules_holding(cls: type, prefix: str) -> list[str]:
    """Loaded modules under `prefix` whose global `RMSNorm` is `cls`."""
    return sorted(name for name, mod in list(sys.modules.items())
                  if name.startswith(prefix) and getattr(mod, "RMSNorm", None) is cls)


def install_rms_norm() -> type:
    """Route vLLM's RMSNorm to DeterministicRMSNorm; returns the replaced class."""
    import vllm.model_executor.layers.layernorm as layernorm
    from vllm.model_executor import custom_op

    from .rms_norm import DeterministicRMSNorm

    replaced = layernorm.RMSNorm
    if replaced is DeterministicRMSNorm:
        return replaced
    DeterministicRMSNorm.name = RMS_NORM_OP_NAME
    custom_op.op_registry[RMS_NORM_OP_NAME] = DeterministicRMSNorm
    custom_op.op_registry_oot[replaced.__name__] = DeterministicRMSNorm
    layernorm.RMSNorm = DeterministicRMSNorm
    stale = _modules_holding(replaced, "vllm.model_executor.models.")
    if stale:
        logger.warning("fxpr_vllm: %d model module(s) imported before the plugin keep vLLM's own "
                       "RMSNorm: %s", len(stale), ", ".join(stale))
    return replaced


def install_attention_backend() -> str:
    """Register the CUSTOM backend by dotted path; returns the path."""
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    register_backend(AttentionBackendEnum.CUSTOM, class_path=BACKEND_CLASS_PATH)
    return BACKEND_CLASS_PATH


# the reference's names
patch_rms_norm = install_rms_norm
patch_attention_backend = install_attention_backend
