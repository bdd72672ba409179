"""vLLM plugin entry point (``vllm.general_plugins``: fxpr_vllm.register:register).

vLLM runs every general plugin in each process it starts, so register() may
run many times per process. It performs the reference plugin's three hooks
(fxpr_vllm/register.py:12-40 of Gursukh/vLLM-Triton-Fixed-Point-Reductions):
the "fixedpoint" quantization config, the CUSTOM attention backend and,
unless FXPR_DISABLE_RMS_NORM=1, the fixed-point RMSNorm. Each hook is a named
step that runs at most once per process; a step that raises is not recorded,
so a later call retries it.
"""

from __future__ import annotations

import logging
from collections.abc import Callable, Iterator

from .config import FxpRuntimeConfig, get_runtime_config

logger = logging.getLogger("fxpr_vllm")

_completed: set[str] = set()


def _install_quant_config() -> None:
    from vllm.model_executor.layers.quantization import register_quantization_config

    from .quantisation_config import FixedPointConfig

    register_quantization_config(FixedPointConfig.get_name())(FixedPointConfig)


def _steps(cfg: FxpRuntimeConfig) -> Iterator[tuple[str, Callable[[], object]]]:
    from . import monkey_patches

    yield "quantization config 'fixedpoint'", _install_quant_config
    yield "attention backend CUSTOM", monkey_patches.install_attention_backend
    if cfg.enable_rms_norm:
        yield "RMSNorm", monkey_patches.install_rms_norm


def register() -> None:
    """Install every enabled hook that has not run in this process yet."""
    cfg = get_runtime_config()
    pending = [(label, step) for label, step in _steps(cfg) if label not in _completed]
    if not pending:
        return
    for label, step in pending:
        step()
        _completed.add(label)
        logger.info("fxpr_vllm: installed %s", label)
    logger.info("fxpr_vllm: Q%d in int%d accumulators; RMSNorm %s, lm_head through gemm_fxp %s",
                cfg.fxp_frac_bits, cfg.fxp_int_bits, "on" if cfg.enable_rms_norm else "off",
                "on" if cfg.enable_lm_head else "off")


def reset_registration() -> None:
    """Forget which hooks ran (tests re-register against a fresh vLLM)."""
    _completed.clear()
