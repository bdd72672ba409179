"""CPU tests of the drop-in boundary: the C-ABI library loads and exports every
entry point include/fxpr.h declares (no compute calls without a GPU), argument
errors come back as codes, the op schemas / fakes match the reference, and the
host-side validation and config logic behave like the reference's."""

from __future__ import annotations

import ctypes
import logging
import pathlib
import re

import pytest
import torch

import fxpr_vllm  # noqa: F401
from fxpr_vllm import _hip, _lib, config
from fxpr_vllm._kernels.fxp import fxp_constants

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fxpr.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(fxpr_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _hip.load()
    names = declared_functions()
    assert "fxpr_gemm" in names or len(names) >= 7
    for name in names:
        assert hasattr(lib, name), f"{name} declared in fxpr.h but not exported"
    # every declared symbol is also bound with a signature on the Python side
    bound = set(_hip.SIGNATURES) | set(_hip.RESTYPES) | {"fxpr_error_string", "fxpr_abi_version"}
    assert set(names) <= bound, set(names) - bound


def test_error_codes_without_gpu():
    lib = _hip.load()
    assert lib.fxpr_abi_version() >= 1
    # argument errors are rejected before any HIP call
    assert lib.fxpr_float_to_fixed(None, 2, None, 24, 16, 10, None) == -2
    assert lib.fxpr_float_to_fixed(None, 2, None, 32, 70, 10, None) == -2
    assert lib.fxpr_float_to_fixed(None, 2, None, 32, 16, -1, None) == -3
    assert lib.fxpr_float_to_fixed(None, 1, ctypes.c_void_p(16), 32, 16, 0, None) == 0  # empty: no-op
    assert lib.fxpr_fixed_to_float(None, 4, None, 8, 16, 10, None) == -2
    assert lib.fxpr_rms_norm(None, None, None, None, 2, 1, 8, 1e-6, None) == -5
    assert lib.fxpr_log_softmax(None, 9, None, 9, 0, 8, 32, 16, None) == 0
    assert "out of range" in _hip.error_string(-2)
    assert _hip.error_string(-4).startswith("fxpr: workspace")


def test_schemas_match_reference():
    # fxpr_vllm/_lib.py:15-33 of the reference, verbatim
    want = {
        "float_to_fixed": "float_to_fixed(Tensor x, int int_bits, int fxp_frac_bits) -> Tensor",
        "fixed_to_float": "fixed_to_float(Tensor x, int float_bits, int fxp_frac_bits) -> Tensor",
        "rms_norm_fxp": "rms_norm_fxp(Tensor x, Tensor weight_fp32, float eps) -> Tensor",
        "rms_norm_fxp_residual": "rms_norm_fxp_residual(Tensor x, Tensor(a!) residual, Tensor weight_fp32, float eps) -> Tensor",
        "gemm_fxp": "gemm_fxp(Tensor a, Tensor b, Tensor? bias, int fxp_int_bits, int fxp_frac_bits) -> Tensor",
        "unified_attention_fxp": (
            "unified_attention_fxp(Tensor q, Tensor kv_cache, Tensor(a!) o, Tensor query_start_loc, "
            "Tensor seq_lens, Tensor block_table, int max_query_len, Tensor? alibi_slopes, bool is_causal, "
            "float? softmax_scale, int fxp_int_bits, int fxp_frac_bits, float logit_softcap, "
            "int window_size, int num_kv_splits) -> ()"),
    }
    for name, schema in want.items():
        got = str(getattr(torch.ops.fxpr, name).default._schema)
        assert got == "fxpr::" + schema, got


def test_fakes_on_meta():
    m = dict(device="meta")
    a = torch.empty(5, 64, dtype=torch.bfloat16, **m)
    b = torch.empty(64, 96, dtype=torch.bfloat16, **m)
    c = torch.ops.fxpr.gemm_fxp(a, b, None, 32, 16)
    assert c.shape == (5, 96) and c.dtype == torch.bfloat16
    x = torch.empty(3, 7, dtype=torch.float16, **m)
    assert torch.ops.fxpr.float_to_fixed(x, 64, 16).dtype == torch.int64
    assert torch.ops.fxpr.fixed_to_float(torch.empty(3, dtype=torch.int32, **m), 16, 16).dtype == torch.float16
    assert torch.ops.fxpr.rms_norm_fxp(x, torch.empty(7, dtype=torch.float16, **m), 1e-6).shape == (3, 7)
    assert torch.ops.fxpr.fixed_row_sum(torch.empty(3, 7, dtype=torch.int16, **m), 64).shape == (3,)
    y = torch.ops.fxpr.log_softmax_fxp(x, 32, 16, torch.float32)
    assert y.shape == (3, 7) and y.dtype == torch.float32


def test_bits_validation_before_any_device_work():
    x = torch.ones(4)
    with pytest.raises(ValueError):
        _lib._float_to_fixed_cuda(x, 12, 16)
    with pytest.raises(ValueError):
        _lib._float_to_fixed_cuda(x, 32, 64)
    with pytest.raises(ValueError):
        _lib._fixed_to_float_cuda(x, 8, 16)
    with pytest.raises(ValueError):
        _lib._log_softmax_fxp_cuda(x, 32, 12)
    # valid bits, but not a device tensor: RuntimeError like the reference
    with pytest.raises(RuntimeError):
        _lib._float_to_fixed_cuda(x, 32, 16)
    with pytest.raises(RuntimeError):
        _lib._rms_norm_fxp_cuda(x.reshape(1, 4), torch.ones(4), 1e-6)


def test_fxp_constants():
    assert fxp_constants(32, 16) == (65536.0, 1.0 / 65536.0, -2147483648.0, 2147483647.0, torch.int32)
    assert fxp_constants(64, 32)[4] == torch.int64
    for bad in ((8, 16), (32, -1), (32, 64)):
        with pytest.raises(ValueError):
            fxp_constants(*bad)


def test_runtime_config_env(monkeypatch, caplog):
    for k in ("FXPR_INT_BITS", "FXPR_FRAC_BITS", "FXPR_DISABLE_RMS_NORM", "FXPR_DISABLE_LM_HEAD"):
        monkeypatch.delenv(k, raising=False)
    cfg = config.load_runtime_config()
    assert (cfg.fxp_int_bits, cfg.fxp_frac_bits, cfg.enable_rms_norm, cfg.enable_lm_head) == (32, 16, True, True)
    monkeypatch.setenv("FXPR_INT_BITS", "64")
    monkeypatch.setenv("FXPR_FRAC_BITS", "32")
    monkeypatch.setenv("FXPR_DISABLE_RMS_NORM", "1")
    cfg = config.load_runtime_config()
    assert (cfg.fxp_int_bits, cfg.fxp_frac_bits, cfg.enable_rms_norm) == (64, 32, False)
    monkeypatch.setenv("FXPR_INT_BITS", "48")
    monkeypatch.setenv("FXPR_FRAC_BITS", "abc")
    with caplog.at_level(logging.WARNING, logger="fxpr_vllm"):
        cfg = config.load_runtime_config()
    assert (cfg.fxp_int_bits, cfg.fxp_frac_bits) == (32, 16)
    assert any("FXPR_INT_BITS" in r.message for r in caplog.records)
    # the cache is per process until reset
    config.reset_runtime_config()
    monkeypatch.setenv("FXPR_INT_BITS", "16")
    assert config.get_runtime_config().fxp_int_bits == 16
    monkeypatch.setenv("FXPR_INT_BITS", "64")
    assert config.get_runtime_config().fxp_int_bits == 16
    config.reset_runtime_config()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_hip, "_lib", None)
    monkeypatch.setattr(_hip, "LIB_PATH", tmp_path / "libfxpr_hip.so")
    with pytest.raises(RuntimeError, match="not built"):
        _hip.load()
