"""Scalar numerics of the fixed-point path, restated in numpy.

Storage conventions: 'f32'/'f64'/'f16' arrays are numpy float32/float64/
float16; 'bf16' arrays are numpy uint16 holding the bfloat16 bit patterns.
All fp32 arithmetic is numpy float32 elementwise arithmetic: one IEEE
round-to-nearest-even per operation, never fused, which is what the HIP
kernels do (they are compiled with -ffp-contract=off).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

INT_DTYPE_BY_BITS = {16: np.int16, 32: np.int32, 64: np.int64}


# ---------------------------------------------------------------------------
# I/O types


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """bfloat16 bits -> float32 (exact)."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round half to even; NaN -> 0x7FC0.

    Same rule as torch's c10::BFloat16 conversion (what `.to(torch.bfloat16)`
    does on the CPU), and as the device helper f32_to_bf16.
    """
    f = np.asarray(f, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
    return np.where(np.isnan(f), np.uint16(0x7FC0), r)


def load(a: np.ndarray, io: str) -> np.ndarray:
    """Storage array -> float32 values (f64 rounds to f32, as the kernels do)."""
    if io == "bf16":
        return bf16_to_f32(a)
    return np.asarray(a).astype(np.float32)


def store(f: np.ndarray, io: str) -> np.ndarray:
    """float32 values -> storage array of the I/O type (RNE)."""
    f = np.asarray(f, dtype=np.float32)
    if io == "bf16":
        return f32_to_bf16(f)
    if io == "f16":
        with np.errstate(over="ignore"):
            return f.astype(np.float16)
    if io == "f32":
        return f.copy()
    if io == "f64":
        return f.astype(np.float64)
    raise ValueError(io)


def round_io(f: np.ndarray, io: str) -> np.ndarray:
    """fl32(IO(f)): round to the I/O type and back."""
    return load(store(f, io), io)


# ---------------------------------------------------------------------------
# Fixed-point casts


def fxp_constants(int_bits: int, frac_bits: int):
    """(scale, inv_scale, qmin, qmax) as the reference computes them.

    Follows fxpr_vllm/_triton/fxp.py:31-53 (fxp_constants): int_bits must be
    16/32/64 and 0 <= frac_bits < 64, else ValueError.
    """
    if int_bits not in (16, 32, 64):
        raise ValueError(f"int_bits must be 16/32/64, got {int_bits}")
    if not (0 <= frac_bits < 64):
        raise ValueError(f"frac_bits must satisfy 0 <= N < 64, got {frac_bits}")
    scale = float(1 << frac_bits)
    return scale, 1.0 / scale, -(1 << (int_bits - 1)), (1 << (int_bits - 1)) - 1


def rne_sat(s: np.ndarray, int_bits: int) -> np.ndarray:
    """Round fp32 values half-to-even, saturate to int_bits, NaN -> 0 (int64).

    This is PTX cvt.rni.sat.s32/.s16.f32 for 32/16 bits and the clamp +
    cvt.rni.s64.f32 sequence for 64 bits (fxpr_vllm/_triton/fxp.py:56-108).
    NaN at 64 bits is not pinned by the reference (it depends on Triton's
    min/max NaN rule); this build defines it as 0 for every width.
    """
    s = np.asarray(s, dtype=np.float32)
    r = np.rint(s).astype(np.float64)  # exact
    lo, hi = -(2.0 ** (int_bits - 1)), 2.0 ** (int_bits - 1)
    nan = np.isnan(r)
    over = r >= hi
    under = r <= lo
    inner = np.where(nan | over | under, 0.0, r)
    q = inner.astype(np.int64)
    q = np.where(over, np.int64((1 << (int_bits - 1)) - 1), q)
    q = np.where(under, np.int64(-(1 << (int_bits - 1))), q)
    return np.where(nan, np.int64(0), q)


def float_to_fixed(x: np.ndarray, int_bits: int, frac_bits: int) -> np.ndarray:
    """q = RNE_sat_b(fl32(x) * 2^f), as an array of the int_bits dtype.

    Follows fxpr_vllm/_triton/fxp.py:92-108 (float_to_fixed) and
    casts.py:21-37, 57-89 (fp16/fp32/fp64 inputs, fp64 rounded to fp32 first).
    """
    scale, _, _, _ = fxp_constants(int_bits, frac_bits)
    x32 = np.asarray(x).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        s = x32 * F32(scale)
    return rne_sat(s, int_bits).astype(INT_DTYPE_BY_BITS[int_bits])


def fixed_to_f32(q: np.ndarray, frac_bits: int) -> np.ndarray:
    """fl32(q) * 2^-f in fp32 (int -> fp32 is a single RNE rounding)."""
    return np.asarray(q).astype(np.float32) * F32(2.0 ** -frac_bits)


def fixed_to_float(q: np.ndarray, float_bits: int, frac_bits: int) -> np.ndarray:
    """OUT(fl32(q) * 2^-f), OUT = f16/f32/f64 for float_bits 16/32/64.

    Follows fxpr_vllm/_triton/fxp.py:111-113 and casts.py:40-54, 92-126: the
    value is always formed in fp32; fp64 output widens it.
    """
    y = fixed_to_f32(q, frac_bits)
    if float_bits == 16:
        with np.errstate(over="ignore"):
            return y.astype(np.float16)
    if float_bits == 32:
        return y
    if float_bits == 64:
        return y.astype(np.float64)
    raise ValueError(f"float_bits must be 16/32/64, got {float_bits}")


def fixed_row_sum(q: np.ndarray, int_bits: int) -> np.ndarray:
    """Exact sum over the last axis, then one saturation to int_bits.

    Follows the fixed-point sum of fxpr_vllm/_tests/test_sum.py:12-16
    (q.sum() in int64, clamp to the int range, cast). Python integers make the
    sum exact for int64 inputs too.
    """
    q = np.asarray(q)
    lo, hi = -(1 << (int_bits - 1)), (1 << (int_bits - 1)) - 1
    flat = q.reshape(-1, q.shape[-1]) if q.ndim else q.reshape(1, 1)
    if q.dtype == np.int64:
        sums = [int(sum(int(v) for v in row)) for row in flat]
    else:
        sums = [int(v) for v in flat.astype(np.int64).sum(axis=1)]
    out = np.array([min(max(s, lo), hi) for s in sums], dtype=INT_DTYPE_BY_BITS[int_bits])
    return out.reshape(q.shape[:-1]) if q.ndim else out.reshape(())


def sat_sum_nonneg(q: np.ndarray, int_bits: int, axis: int = -1) -> np.ndarray:
    """Sum of non-negative fixed-point terms, clamped once to the int_bits max.

    For terms in [0, qmax] this equals every saturating reduction tree, which
    is what the kernels compute. Exact via Python ints when int64 could wrap.
    """
    q = np.asarray(q, dtype=np.int64)
    hi = (1 << (int_bits - 1)) - 1
    if int_bits < 64 and q.shape[axis] < (1 << 31):
        s = q.sum(axis=axis)
        return np.minimum(s, hi)
    moved = np.moveaxis(q, axis, -1)
    flat = moved.reshape(-1, moved.shape[-1])
    sums = [min(sum(int(v) for v in row), hi) for row in flat]
    return np.array(sums, dtype=np.int64).reshape(moved.shape[:-1])


def int_to_f32(n: int) -> np.float32:
    """fl32 of a non-negative Python integer of any size: round half to even
    to 24 significant bits (inf beyond the fp32 range)."""
    n = int(n)
    if n < 0:
        raise ValueError("int_to_f32 takes non-negative integers")
    sh = n.bit_length() - 24
    if sh > 0:
        q, rem = divmod(n, 1 << sh)
        half = 1 << (sh - 1)
        if rem > half or (rem == half and q & 1):
            q += 1
        n = q << sh
    with np.errstate(over="ignore"):
        return np.float32(float(n)) if n < 2 ** 128 else np.float32(np.inf)


def exact_sum_nonneg_f32(q: np.ndarray, axis: int = -1) -> tuple[np.ndarray, np.ndarray]:
    """(S == 0, fl32(S)) for S the exact sum of non-negative int64 terms along
    `axis`; numpy int64 sums where they cannot wrap, Python integers beyond."""
    q = np.asarray(q, dtype=np.int64)
    moved = np.moveaxis(q, axis, -1)
    flat = moved.reshape(-1, moved.shape[-1])
    n = flat.shape[-1]
    top = int(flat.max()) if flat.size else 0
    if top * n < (1 << 63):
        s = flat.sum(axis=-1)
        zero, f = s == 0, s.astype(np.float32)
    else:
        sums = [sum(int(v) for v in row) for row in flat]
        zero = np.array([t == 0 for t in sums], dtype=bool)
        f = np.array([int_to_f32(t) for t in sums], dtype=np.float32)
    return zero.reshape(moved.shape[:-1]), f.reshape(moved.shape[:-1])


# ---------------------------------------------------------------------------
# The build's own exp and log (no reference counterpart: the reference's
# log-softmax file is absent, fxpr_vllm README.md:60). Cody-Waite style
# reduction to a power of two plus a Taylor polynomial by Horner's rule (exp:
# fused multiply-adds; log: separate products and sums), one fp32 rounding per
# operation; the device restatement is csrc/fxp_device.h.

EXP2_C = [F32(c) for c in (
    1.0,
    0.693147180559945309,
    0.240226506959100712,
    0.0555041086648215800,
    0.00961812910762847717,
    0.00133335581464284434,
    0.000154035303933816099,
    1.52527338040598403e-05,
)]
LOG2E = F32(1.44269504088896341)
LN2_HI = F32(0.693145751953125)
LN2_LO = F32(1.42860682030941723e-06)
SQRT2 = F32(1.41421356237309505)
EXP_FLOOR = F32(-80.0)
LOG_C = [F32(c) for c in (1.0, 1.0 / 3.0, 0.2, 1.0 / 7.0, 1.0 / 9.0)]


def fma_f32(a, b, c) -> np.ndarray:
    """fl32(a * b + c) with one rounding (round half to even): IEEE fused
    multiply-add on fp32 operands.

    The product of two fp32 values is exact in float64; the float64 sum s is
    completed by its exact error e (TwoSum), so s + e = a*b + c exactly.
    Rounding s to fp32 gives the correctly rounded result unless s lies
    exactly half-way between two fp32 neighbours while e != 0: the tie then
    goes to the neighbour on e's side. (|e| is at most half a float64 ulp of
    s, far below half an fp32 ulp, so no other case can differ.)"""
    a64 = np.asarray(a, dtype=np.float32).astype(np.float64)
    b64 = np.asarray(b, dtype=np.float32).astype(np.float64)
    c64 = np.asarray(c, dtype=np.float32).astype(np.float64)
    p = a64 * b64
    with np.errstate(invalid="ignore", over="ignore"):
        s = p + c64
        bv = s - p
        e = (p - (s - bv)) + (c64 - bv)
        r = s.astype(np.float32)
        r64 = r.astype(np.float64)
        up = np.nextafter(r, np.float32(np.inf)).astype(np.float64)
        dn = np.nextafter(r, np.float32(-np.inf)).astype(np.float64)
        tie_up = (s == (r64 + up) * 0.5) & (e > 0)   # true sum just above an upper tie
        tie_dn = (s == (r64 + dn) * 0.5) & (e < 0)   # true sum just below a lower tie
    fin = np.isfinite(s) & np.isfinite(e)
    out = np.where(fin & tie_up, up, np.where(fin & tie_dn, dn, r64))
    return out.astype(np.float32)


def exp2_poly(r: np.ndarray) -> np.ndarray:
    """2^r for |r| <= 0.5: degree-7 Taylor polynomial, Horner's rule with
    fused multiply-adds (one rounding per step)."""
    r = np.asarray(r, dtype=np.float32)
    p = np.full_like(r, EXP2_C[7])
    for c in EXP2_C[6::-1]:
        p = fma_f32(p, r, c)
    return p


def exp_scaled(d: np.ndarray, frac_bits: int) -> np.ndarray:
    """fl32(exp_own(d) * 2^f) for d <= 0; 0 where d < -80 or d is NaN."""
    d = np.asarray(d, dtype=np.float32)
    ok = d >= EXP_FLOOR
    dd = np.where(ok, d, F32(0.0))
    t = dd * LOG2E
    k = np.rint(t)
    r = t - k
    p = exp2_poly(r)
    out = np.ldexp(p, (k.astype(np.int32) + np.int32(frac_bits)))
    return np.where(ok, out, F32(0.0)).astype(np.float32)


def log_own(y: np.ndarray) -> np.ndarray:
    """ln(y) for positive normal fp32 y (see csrc/fxp_device.h log_own)."""
    y = np.asarray(y, dtype=np.float32)
    bits = y.view(np.uint32)
    e = (bits >> np.uint32(23)).astype(np.int32) - np.int32(127)
    m = ((bits & np.uint32(0x007FFFFF)) | np.uint32(0x3F800000)).view(np.float32)
    big = m > SQRT2
    m = np.where(big, m * F32(0.5), m)
    e = np.where(big, e + 1, e)
    s = (m - F32(1.0)) / (m + F32(1.0))
    z = s * s
    p = np.full_like(z, LOG_C[4])
    for c in LOG_C[3::-1]:
        p = p * z + c
    lnm = (s * F32(2.0)) * p
    fe = e.astype(np.float32)
    return fe * LN2_HI + (fe * LN2_LO + lnm)
