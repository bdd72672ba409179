"""Helpers shared by the tests: torch <-> oracle storage conversion."""

from __future__ import annotations

import numpy as np
import torch

IO_NAME = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32", torch.float64: "f64"}


def to_np(t: torch.Tensor) -> np.ndarray:
    """Tensor -> numpy storage as the oracle expects (bf16 as uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def from_np(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """Oracle storage -> CPU tensor of `dtype`."""
    if dtype == torch.bfloat16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype)


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality (NaN == NaN when the bit patterns match)."""
    a = a.detach().cpu().contiguous()
    b = b.detach().cpu().contiguous()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.is_floating_point():
        view = {2: torch.int16, 4: torch.int32, 8: torch.int64}[a.element_size()]
        return torch.equal(a.view(view), b.view(view))
    return torch.equal(a, b)


def nan_aware_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Equal values, any NaN matching any NaN (payloads may differ)."""
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    if a.shape != b.shape:
        return False
    both_nan = torch.isnan(a) & torch.isnan(b)
    return bool(torch.all(both_nan | (a == b)))


def mismatch_report(got: torch.Tensor, want: torch.Tensor, k: int = 5) -> str:
    g = got.detach().cpu().double().reshape(-1)
    w = want.detach().cpu().double().reshape(-1)
    bad = torch.nonzero(~((g == w) | (torch.isnan(g) & torch.isnan(w)))).reshape(-1)
    idx = bad[:k].tolist()
    return f"{bad.numel()} mismatches; first {[(i, g[i].item(), w[i].item()) for i in idx]}"


def seeded(shape, seed: int, std: float = 1.0, mean: float = 0.0, dtype=torch.float32):
    """Seeded CPU normal data (the bench and tests generate on the CPU, then copy)."""
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std + mean).to(dtype)


def close_report(got: torch.Tensor, want: torch.Tensor, rtol: float = 1e-2, atol_rms: float = 1e-3) -> str:
    """'' when every element satisfies |got - want| <= rtol * |want| + atol,
    with atol = atol_rms * RMS(want) (a floor for outputs near zero, where a
    relative bound means nothing); else a description of the worst element.

    rtol = 1e-2 is the north star's "within 1e-2 relative" for the GEMM and
    attention paths. Non-finite values must match exactly."""
    g = got.detach().cpu().double().reshape(-1)
    w = want.detach().cpu().double().reshape(-1)
    if g.shape != w.shape:
        return f"shape {tuple(got.shape)} != {tuple(want.shape)}"
    fin = torch.isfinite(w)
    same_nonfinite = (torch.isnan(g) & torch.isnan(w)) | (g == w)
    if not bool(torch.all(fin | same_nonfinite)):
        return "non-finite values differ"
    g, w = g[fin], w[fin]
    if w.numel() == 0:
        return ""
    atol = atol_rms * float(torch.sqrt((w * w).mean()))
    excess = (g - w).abs() - (rtol * w.abs() + atol)
    i = int(torch.argmax(excess))
    if excess[i] <= 0:
        return ""
    return (f"{int((excess > 0).sum())} elements out of tolerance; worst: got {g[i].item()!r} want "
            f"{w[i].item()!r} (rtol {rtol}, atol {atol:.3g})")
