"""Row reductions: RMSNorm(+residual) and log-softmax, restated in numpy."""

from __future__ import annotations

import numpy as np

from .numerics import (
    F32,
    exp_scaled,
    fixed_to_f32,
    load,
    log_own,
    rne_sat,
    round_io,
    sat_sum_nonneg,
    store,
)


def rms_norm(x, w, eps, io, int_bits, frac_bits, residual=None):
    """Deterministic RMSNorm over the last axis; returns (y, new_residual).

    Op order and rounding points follow fxpr_vllm/_triton/rms_norm.py:38-64:
    v = fl32(x) [+ fl32(r)], the residual is stored as IO(v) (:45-48),
    mean_sq = max(acc / H, 0) (:52), rrms from mean_sq + eps (:53),
    pass 2 re-reads the stored residual (IO-rounded v) or x (:58-61),
    y = IO((u * w) * rrms) (:63-64).
    Differences this build defines (the reference sums v*v in fp32 in an
    unspecified order, :49-50; its rsqrt is libdevice, :53):
      acc = fl32(sat_sum(float_to_fixed(fl32(v*v), int_bits, frac_bits))) * 2^-f
      rrms = fl32(1 / fl32(sqrt(fl32(mean_sq + eps))))   (IEEE sqrt, division)
    so the bits are fixed for any reduction order.
    """
    x = np.asarray(x)
    shape = x.shape
    H = shape[-1]
    xf = load(x, io).reshape(-1, H)
    wf = load(np.asarray(w), io).reshape(H)
    if residual is not None:
        v = xf + load(np.asarray(residual), io).reshape(-1, H)
        new_r = store(v, io)
        u = load(new_r, io)
    else:
        v = xf
        new_r = None
        u = xf
    sq = v * v
    with np.errstate(over="ignore", invalid="ignore"):
        q = rne_sat(sq * F32(2.0 ** frac_bits), int_bits)
    total = sat_sum_nonneg(q, int_bits, axis=1)
    acc = fixed_to_f32(total, frac_bits)
    ms = acc / F32(H)
    ms = np.maximum(ms, F32(0.0))
    rrms = F32(1.0) / np.sqrt(ms + F32(eps))
    y = store((u * wf[None, :]) * rrms[:, None], io).reshape(shape)
    if new_r is not None:
        new_r = new_r.reshape(shape)
    return y, new_r


def log_softmax(x, io_in, io_out, int_bits, frac_bits):
    """Deterministic log-softmax over the last axis.

    Build-defined semantics (the reference lists _triton/softmax.py in its
    README, fxpr_vllm README.md:60, but ships no file): m = max_j fl32(x_j)
    (NaN propagates); S = sat_sum_j RNE_sat(exp_scaled(fl32(x_j) - m, f));
    lse = m + log_own(fl32(S) * 2^-f) (S = 0 gives -inf);
    y_j = OUT(fl32(x_j) - lse). The denominator is modelled on the reference
    attention denominator, which quantises each exp weight and sums integers
    (fxpr_vllm/_triton/attention.py:285-286, 608-610).
    """
    x = np.asarray(x)
    shape = x.shape
    V = shape[-1]
    xf = load(x, io_in).reshape(-1, V)
    with np.errstate(invalid="ignore"):
        m = np.max(xf, axis=1)  # numpy max propagates NaN
        d = xf - m[:, None]
    e = exp_scaled(d, frac_bits)
    q = rne_sat(e, int_bits)
    total = sat_sum_nonneg(q, int_bits, axis=1)
    S = fixed_to_f32(total, frac_bits)
    with np.errstate(divide="ignore", invalid="ignore"):
        lnS = np.where(total == 0, F32(-np.inf), log_own(np.where(total == 0, F32(1.0), S)))
        lse = (m + lnS).astype(np.float32)
        y = xf - lse[:, None]
    return store(y, io_out).reshape(shape)


def rms_norm_reference_fp32(x, w, eps, residual=None):
    """The reference's own test model of RMSNorm in fp32 (tolerance checks).

    fxpr_vllm/_tests/test_rms_norm.py:18-28: mean_sq = mean(x*x),
    rrms = 1/sqrt(mean_sq + eps), y = x * w * rrms.
    """
    x = np.asarray(x, dtype=np.float64)
    if residual is not None:
        x = x + np.asarray(residual, dtype=np.float64)
    ms = (x * x).mean(axis=-1, keepdims=True)
    return x * np.asarray(w, dtype=np.float64) / np.sqrt(ms + eps)


__all__ = ["rms_norm", "log_softmax", "rms_norm_reference_fp32", "round_io"]
