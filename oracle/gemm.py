"""Fixed-point GEMM, restated in numpy."""

from __future__ import annotations

import numpy as np

from .numerics import F32, fixed_to_f32, load, rne_sat, store

BLOCK_K = {"bf16": 128, "f16": 128, "f32": 64}


def wrap_bits(v: np.ndarray, int_bits: int) -> np.ndarray:
    """Two's-complement wrap of int64 values to int_bits (as int64)."""
    v = np.asarray(v, dtype=np.int64)
    if int_bits == 64:
        return v
    m = np.int64(1 << int_bits)
    h = np.int64(1 << (int_bits - 1))
    return ((v + h) % m) - h


def gemm(a, b, bias, io, int_bits, frac_bits, block_k=None):
    """C = IO(fl32(acc) * 2^-f (+ fl32(bias))), acc = wrapping sum over K-tiles
    of RNE_sat(fl32(partial) * 2^f).

    Follows fxpr_vllm/_triton/gemm.py:183-204 (persistent kernel body): per
    BLOCK_K tile an fp32 dot partial is quantised with float_to_fixed and
    added into an int accumulator of int_bits (wrapping add, :190); the tail
    tile is zero-padded (:185-187); epilogue fixed_to_float, + fp32 bias, cast
    to the I/O dtype (:195-204). BLOCK_K is 128 for bf16/f16 and 64 for fp32
    (:26-30).
    Parity unpinned at the bit level for general inputs: the order in which a
    tile's 128 products are added in fp32 is the hardware's (NVIDIA mma in the
    reference, MFMA on MI355X, BLAS sgemm here), so general inputs are checked
    to a tolerance; inputs whose tile dots are exact in fp32 (small integers)
    are checked bit for bit. The oracle's own tile partial is the float64 dot
    (every product of two bf16/f16/f32 values is exact in float64) rounded
    once to fp32: independent of operand layout and summation order.
    """
    af = load(np.asarray(a), io).astype(np.float64)
    bf = load(np.asarray(b), io).astype(np.float64)
    M, K = af.shape
    N = bf.shape[1]
    bk = block_k or BLOCK_K[io]
    acc = np.zeros((M, N), dtype=np.int64)
    scale = F32(2.0 ** frac_bits)
    with np.errstate(over="ignore", invalid="ignore"):
        for t in range(0, K, bk):
            p = (af[:, t:t + bk] @ bf[t:t + bk, :]).astype(np.float32)
            q = rne_sat(p * scale, int_bits)
            acc = acc + q  # int64 arithmetic wraps; reduced to int_bits below
    acc = wrap_bits(acc, int_bits)
    c = fixed_to_f32(acc, frac_bits)
    if bias is not None:
        c = c + load(np.asarray(bias), io if np.asarray(bias).dtype != np.float32 else "f32").reshape(1, N)
    return store(c.astype(np.float32), io)
