"""Row reductions: RMSNorm(+residual) and log-softmax, restated in numpy."""

from __future__ import annotations

import numpy as np

from .numerics import (
    F32,
    exact_sum_nonneg_f32,
    exp_scaled,
    load,
    log_own,
    rne_sat,
    round_io,
    store,
)


# Fraction bits of the RMSNorm sum-of-squares terms below the row's scale:
# every term (v * 2^-e)^2 is below 4, so a 64-bit unsigned sum of rows up to
# 2^22 elements cannot wrap, and a term below 2^-41 of the row maximum's
# square (far under fp32's own 2^-24 resolution) is what rounds away.
RMS_SUM_FRAC = 40
RMS_MAX_HIDDEN = 1 << 22


def rms_row_exponent(v):
    """Per row, e with 2^e <= max_j |v_j| < 2^(e+1) (e = -126 when the row's
    maximum is zero or subnormal), and the row maximum's magnitude bits."""
    bits = np.asarray(v, dtype=np.float32).view(np.uint32) & np.uint32(0x7FFFFFFF)
    mbits = bits.max(axis=-1)
    biased = (mbits >> np.uint32(23)).astype(np.int32)
    e = np.maximum(biased, 1) - 127
    return e, mbits


def rms_norm(x, w, eps, io, residual=None):
    """Deterministic RMSNorm over the last axis; returns (y, new_residual).

    Op order and rounding points follow fxpr_vllm/_triton/rms_norm.py:38-64:
    v = fl32(x) [+ fl32(r)], the residual is stored as IO(v) (:45-48),
    mean_sq from the sum of v*v over the unrounded v (:49-52), rrms from
    mean_sq + eps (:53), pass 2 re-reads the stored residual (IO-rounded v) or
    x (:58-61), y = IO((u * w) * rrms) (:63-64).

    The reference sums v*v in fp32 in an unspecified order (:49-50); this
    build sums integers, so the bits are fixed for any reduction order, in a
    per-row block floating-point format that cannot overflow:
      e   = exponent of max_j |v_j| (rms_row_exponent)
      s_j = fl32(ldexp(v_j, -e))                      (|s_j| < 2)
      q_j = RNE(fl32(s_j * s_j) * 2^40)               (< 2^42, exact in f64)
      T   = exact 64-bit sum of q_j
      mean_sq = ldexp(fl32(fl32(T) / fl32(H)), 2e - 40)   (one rounding each)
      rrms = fl32(1 / fl32(sqrt(fl32(mean_sq + eps))))    (IEEE sqrt, division)
    A row whose maximum is inf or NaN takes mean_sq = that maximum (inf or
    NaN), as the reference's fp32 sum would. The format does not depend on the
    FXPR_INT_BITS / FXPR_FRAC_BITS knobs (the reference's RMSNorm takes none).
    """
    x = np.asarray(x)
    shape = x.shape
    H = shape[-1]
    if H > RMS_MAX_HIDDEN:
        raise ValueError(f"rms_norm: hidden size {H} exceeds {RMS_MAX_HIDDEN}")
    xf = load(x, io).reshape(-1, H)
    wf = load(np.asarray(w), io).reshape(H)
    if residual is not None:
        with np.errstate(over="ignore", invalid="ignore"):
            v = xf + load(np.asarray(residual), io).reshape(-1, H)
        new_r = store(v, io)
        u = load(new_r, io)
    else:
        v = xf
        new_r = None
        u = xf
    e, mbits = rms_row_exponent(v)
    finite = mbits < np.uint32(0x7F800000)
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        s = np.ldexp(v, (-e)[:, None]).astype(np.float32)
        t = (s * s).astype(np.float32)
    t = np.where(finite[:, None], t, F32(0.0))
    q = np.rint(t.astype(np.float64) * 2.0 ** RMS_SUM_FRAC).astype(np.uint64)
    total = q.sum(axis=1, dtype=np.uint64)
    with np.errstate(over="ignore", under="ignore"):
        mean_scaled = (total.astype(np.float32) / F32(H)).astype(np.float32)
        ms = np.ldexp(mean_scaled, 2 * e - RMS_SUM_FRAC).astype(np.float32)
    ms = np.where(finite, ms, mbits.view(np.float32))
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        rrms = F32(1.0) / np.sqrt(ms + F32(eps))
        y = store((u * wf[None, :]) * rrms[:, None], io).reshape(shape)
    if new_r is not None:
        new_r = new_r.reshape(shape)
    return y, new_r


def log_softmax(x, io_in, io_out, int_bits, frac_bits):
    """Deterministic log-softmax over the last axis.

    Build-defined semantics (the reference lists _triton/softmax.py in its
    README, fxpr_vllm README.md:60, but ships no file): m = max_j fl32(x_j)
    (NaN propagates); q_j = RNE_sat_b(exp_scaled(fl32(x_j) - m, f)); S = the
    exact sum of the q_j (a wide integer: it never saturates, so near-flat
    full-vocabulary rows normalise); lse = m + log_own(fl32(S) * 2^-f) with
    fl32(S) correctly rounded (S = 0 gives -inf); y_j = OUT(fl32(x_j) - lse).
    The denominator is modelled on the reference attention denominator, which
    quantises each exp weight and sums integers
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
    zero, S32 = exact_sum_nonneg_f32(q, axis=1)
    S = (S32 * F32(2.0 ** -frac_bits)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        lnS = np.where(zero, F32(-np.inf), log_own(np.where(zero, F32(1.0), S)))
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
