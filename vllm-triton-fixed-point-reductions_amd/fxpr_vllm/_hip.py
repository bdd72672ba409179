"""ctypes binding of libfxpr_hip.so (declarations: include/fxpr.h).

The library is loaded on first use. If it is missing the call raises
RuntimeError: there is no CPU or Triton fallback behind these ops.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libfxpr_hip.so")

DTYPE_CODE = {
    torch.float16: 0,
    torch.bfloat16: 1,
    torch.float32: 2,
    torch.float64: 3,
    torch.int16: 4,
    torch.int32: 5,
    torch.int64: 6,
}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

# name -> argtypes (every entry point returns int)
SIGNATURES: dict[str, list] = {
    "fxpr_float_to_fixed": [_P, _I, _P, _I, _I, _L, _P],
    "fxpr_fixed_to_float": [_P, _I, _P, _I, _I, _L, _P],
    "fxpr_fixed_row_sum": [_P, _I, _P, _I, _L, _L, _P],
    "fxpr_rms_norm": [_P, _P, _P, _P, _I, _L, _L, _F, _P],
    "fxpr_log_softmax": [_P, _I, _P, _I, _L, _L, _I, _I, _P],
    "fxpr_log_softmax_shard_max": [_P, _I, _P, _L, _L, _P],
    "fxpr_log_softmax_shard_sum": [_P, _I, _P, _P, _L, _L, _I, _I, _P],
    "fxpr_log_softmax_shard_finish": [_P, _I, _P, _P, _P, _I, _L, _L, _I, _P],
    "fxpr_sample_greedy": [_P, _I, _L, _L, _I, _I, _I, _P, _P, _P, _P, _P, _L, _P],
    "fxpr_gemm": [_P, _P, _P, _P, _I, _L, _L, _L, _L, _L, _L, _L, _L, _L, _I, _I, _I, _P, _L, _P],
    "fxpr_gemm_splits": [_L, _L, _L, _I, _I, _I],
    "fxpr_gemm_partial": [_P, _P, _P, _I, _L, _L, _L, _L, _L, _L, _L, _I, _I, _P],
    "fxpr_gemm_finish": [_P, _P, _P, _I, _L, _L, _L, _L, _I, _I, _P],
    "fxpr_unified_attention": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _L, _I, _I, _I, _I, _I, _I, _L,
                               _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L,
                               _I, _F, _F, _I, _I, _I, _I, _P, _L, _P],
    "fxpr_unified_attention_noalloc": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _L, _I, _I, _I, _I, _I, _I, _L,
                                       _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L,
                                       _I, _F, _F, _I, _I, _I, _I, _P],
    "fxpr_attention_splits": [_I, _I, _I, _I, _I, _I, _I],
    "fxpr_reshape_and_cache": [_P, _P, _P, _P, _I, _P, _L, _I, _I, _I, _L,
                               _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _P],
    # test hooks of the split log-softmax's bounded polls
    "fxpr_debug_set_lsm_spin_limit": [_I, _I],
    "fxpr_debug_lsm_default_spin_limit": [],
    "fxpr_debug_lsm_fallbacks": [ctypes.POINTER(ctypes.c_ulonglong)],
}

# entry points that return something other than an int status
RESTYPES = {
    "fxpr_gemm_workspace_bytes": ([_L, _L, _L, _I, _I, _I], _L),
    "fxpr_attention_workspace_bytes": ([_I, _L, _I, _I, _I, _I, _I, _I, _I, _I], _L),
    "fxpr_sample_greedy_workspace_bytes": ([_L, _I], _L),
}

# the ABI revision these signatures describe (include/fxpr.h, fxpr_abi_version)
ABI_VERSION = 3

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load and declare the library (idempotent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"fxpr: HIP kernel library not built ({LIB_PATH}); run "
                    "`python build.py` in the package directory (or "
                    "__graft_entry__.build())"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.fxpr_error_string.argtypes = [_I]
            lib.fxpr_error_string.restype = ctypes.c_char_p
            lib.fxpr_abi_version.argtypes = []
            lib.fxpr_abi_version.restype = _I
            if lib.fxpr_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"fxpr: {LIB_PATH} implements ABI revision {lib.fxpr_abi_version()}, these bindings "
                    f"revision {ABI_VERSION}; rebuild it (`python build.py` in the package directory)"
                )
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _I
            for name, (argtypes, restype) in RESTYPES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = lib
    return _lib


def error_string(code: int) -> str:
    return load().fxpr_error_string(int(code)).decode()


def call(name: str, *args) -> None:
    """Call an entry point; raise RuntimeError on a non-zero return."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed: {error_string(rc)} (code {rc})")


def stream_ptr(device: torch.device) -> int:
    """Handle of the current torch stream on `device` (launch target)."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
