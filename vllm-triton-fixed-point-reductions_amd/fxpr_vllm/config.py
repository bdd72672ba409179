"""Process-wide settings of the fixed-point plugin, read from the environment.

The variables, their accepted values and defaults are the reference plugin's
(fxpr_vllm/config.py:6-73 of Gursukh/vLLM-Triton-Fixed-Point-Reductions), so
a deployment configured for it behaves the same here:

    variable                         accepted              default
    FXPR_INT_BITS                    16 | 32 | 64          32
    FXPR_FRAC_BITS                   8 | 16 | 32           16
    FXPR_DISABLE_RMS_NORM            "1" = keep vLLM's RMSNorm
    FXPR_DISABLE_LM_HEAD             "1" = keep vLLM's lm_head matmul
    FXPR_DISABLE_ATTENTION_WARMUP    "1" = no attention warm-up at first use
    FXPR_DISABLE_GEMM_WARMUP         "1" = no GEMM warm-up at weight load
    FXPR_DISABLE_RMS_NORM_WARMUP     "1" = no RMSNorm warm-up at weight load

A value that does not parse or is not accepted is logged on the "fxpr_vllm"
logger and replaced by the default: a mistyped knob must not keep a serving
process from starting. The knobs set the fixed-point format of the GEMM,
attention and log-softmax paths; RMSNorm has a format of its own.

The settings are read on first use and cached for the life of the process
(vLLM starts one process per GPU); reset_runtime_config() drops the cache.
"""

from __future__ import annotations

import functools
import logging
import os
from collections.abc import Mapping
from dataclasses import dataclass

DEFAULT_FXP_INT_BITS = 32
DEFAULT_FXP_FRAC_BITS = 16

logger = logging.getLogger("fxpr_vllm")


@dataclass(frozen=True)
class FxpRuntimeConfig:
    """The resolved settings (field names are the reference's)."""

    fxp_int_bits: int = DEFAULT_FXP_INT_BITS
    fxp_frac_bits: int = DEFAULT_FXP_FRAC_BITS
    enable_rms_norm: bool = True
    enable_lm_head: bool = True
    disable_attention_warmup: bool = False
    disable_gemm_warmup: bool = False
    disable_rms_norm_warmup: bool = False


@dataclass(frozen=True)
class _IntChoice:
    """An integer knob restricted to a fixed set of values."""

    var: str
    accepted: tuple[int, ...]
    default: int

    def resolve(self, environ: Mapping[str, str]) -> int:
        text = environ.get(self.var, "").strip()
        if not text:
            return self.default
        try:
            value = int(text, 10)
        except ValueError:
            value = None
        if value in self.accepted:
            return value
        logger.warning("%s=%r is not one of %s; falling back to %d", self.var, text,
                       "/".join(str(v) for v in self.accepted), self.default)
        return self.default


_CHOICES = {
    "fxp_int_bits": _IntChoice("FXPR_INT_BITS", (16, 32, 64), DEFAULT_FXP_INT_BITS),
    "fxp_frac_bits": _IntChoice("FXPR_FRAC_BITS", (8, 16, 32), DEFAULT_FXP_FRAC_BITS),
}

# field -> variable whose value "1" flips the field away from its default
_SWITCHES = {
    "enable_rms_norm": "FXPR_DISABLE_RMS_NORM",
    "enable_lm_head": "FXPR_DISABLE_LM_HEAD",
    "disable_attention_warmup": "FXPR_DISABLE_ATTENTION_WARMUP",
    "disable_gemm_warmup": "FXPR_DISABLE_GEMM_WARMUP",
    "disable_rms_norm_warmup": "FXPR_DISABLE_RMS_NORM_WARMUP",
}


def load_runtime_config(environ: Mapping[str, str] | None = None) -> FxpRuntimeConfig:
    """Resolve every knob from `environ` (default: the process environment)."""
    env = os.environ if environ is None else environ
    defaults = FxpRuntimeConfig()
    fields: dict[str, object] = {name: c.resolve(env) for name, c in _CHOICES.items()}
    for name, var in _SWITCHES.items():
        flipped = env.get(var, "").strip() == "1"
        fields[name] = (not getattr(defaults, name)) if flipped else getattr(defaults, name)
    return FxpRuntimeConfig(**fields)


@functools.lru_cache(maxsize=1)
def get_runtime_config() -> FxpRuntimeConfig:
    """The process's settings, resolved once."""
    return load_runtime_config()


def reset_runtime_config() -> None:
    """Drop the cached settings; the next get_runtime_config() re-reads the environment."""
    get_runtime_config.cache_clear()
