"""Process-wide knobs, read once from the environment.

Same variables, defaults and fallbacks as the reference plugin
(fxpr_vllm/config.py:11-73 of Gursukh/vLLM-Triton-Fixed-Point-Reductions):

    FXPR_INT_BITS                  16 / 32 / 64 (default 32), else warn + default
    FXPR_FRAC_BITS                 8 / 16 / 32 (default 16), else warn + default
    FXPR_DISABLE_RMS_NORM=1        keep vLLM's stock RMSNorm
    FXPR_DISABLE_LM_HEAD=1         keep vLLM's lm_head matmul
    FXPR_DISABLE_ATTENTION_WARMUP=1, FXPR_DISABLE_GEMM_WARMUP=1,
    FXPR_DISABLE_RMS_NORM_WARMUP=1 skip the load-time warm-up calls

RMSNorm and log-softmax take their fixed-point format from FXPR_INT_BITS /
FXPR_FRAC_BITS, since their schemas carry no bit arguments.
"""

from __future__ import annotations

import logging
import os
from dataclasses import dataclass

DEFAULT_FXP_INT_BITS = 32
DEFAULT_FXP_FRAC_BITS = 16

logger = logging.getLogger("fxpr_vllm")


def _read_int(name: str, default: int) -> int:
    raw = os.environ.get(name)
    if raw is None or raw == "":
        return default
    try:
        return int(raw)
    except ValueError:
        logger.warning("Ignoring malformed %s=%r; using default %d", name, raw, default)
        return default


def _flag(name: str) -> bool:
    return os.environ.get(name) == "1"


@dataclass(frozen=True)
class FxpRuntimeConfig:
    fxp_int_bits: int = DEFAULT_FXP_INT_BITS
    fxp_frac_bits: int = DEFAULT_FXP_FRAC_BITS
    enable_rms_norm: bool = True
    enable_lm_head: bool = True
    disable_attention_warmup: bool = False
    disable_gemm_warmup: bool = False
    disable_rms_norm_warmup: bool = False


def load_runtime_config() -> FxpRuntimeConfig:
    int_bits = _read_int("FXPR_INT_BITS", DEFAULT_FXP_INT_BITS)
    if int_bits not in (16, 32, 64):
        logger.warning("Invalid FXPR_INT_BITS=%d; must be 16/32/64. Using default %d.",
                       int_bits, DEFAULT_FXP_INT_BITS)
        int_bits = DEFAULT_FXP_INT_BITS
    frac_bits = _read_int("FXPR_FRAC_BITS", DEFAULT_FXP_FRAC_BITS)
    if frac_bits not in (8, 16, 32):
        logger.warning("Invalid FXPR_FRAC_BITS=%d; must be 8/16/32. Using default %d.",
                       frac_bits, DEFAULT_FXP_FRAC_BITS)
        frac_bits = DEFAULT_FXP_FRAC_BITS
    return FxpRuntimeConfig(
        fxp_int_bits=int_bits,
        fxp_frac_bits=frac_bits,
        enable_rms_norm=not _flag("FXPR_DISABLE_RMS_NORM"),
        enable_lm_head=not _flag("FXPR_DISABLE_LM_HEAD"),
        disable_attention_warmup=_flag("FXPR_DISABLE_ATTENTION_WARMUP"),
        disable_gemm_warmup=_flag("FXPR_DISABLE_GEMM_WARMUP"),
        disable_rms_norm_warmup=_flag("FXPR_DISABLE_RMS_NORM_WARMUP"),
    )


_runtime_config: FxpRuntimeConfig | None = None


def get_runtime_config() -> FxpRuntimeConfig:
    global _runtime_config
    if _runtime_config is None:
        _runtime_config = load_runtime_config()
    return _runtime_config


def reset_runtime_config() -> None:
    """Forget the cached config so the next call re-reads the environment."""
    global _runtime_config
    _runtime_config = None
