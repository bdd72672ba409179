"""Greedy sampling with log-probabilities, restated in numpy.

Build-defined (the reference lists fxpr_vllm/sampling.py in README.md:69
but ships no file). Per row: the order is largest fl32 value first, equal
values by ascending index, every NaN above +inf, -0 equal to +0. The sampled
token is the first element of the order; the top-k are the first k; every
log-probability is rows.log_softmax's fp32 output at that element (the same
lse, hence the same bits).
"""

from __future__ import annotations

import numpy as np

from .numerics import load
from .rows import log_softmax


def value_order(xf: np.ndarray) -> np.ndarray:
    """uint32 order of fp32 values: larger value -> larger; -0 == +0; NaN on top."""
    xf = np.asarray(xf, dtype=np.float32)
    u = np.where(xf == 0, np.uint32(0), xf.view(np.uint32)).astype(np.uint32)
    neg = (u & np.uint32(0x80000000)) != 0
    key = np.where(neg, ~u, u | np.uint32(0x80000000)).astype(np.uint32)
    return np.where(np.isnan(xf), np.uint32(0xFFFFFFFF), key)


def sample_greedy(x, io, num_logprobs, int_bits, frac_bits):
    """(ids [R], logprobs [R], topk_ids [R, k], topk_logprobs [R, k]) for x [R, V]."""
    x = np.asarray(x)
    V = x.shape[-1]
    xf = load(x, io).reshape(-1, V)
    y = log_softmax(x, io, "f32", int_bits, frac_bits).reshape(-1, V)
    idx = np.arange(V, dtype=np.uint64)
    keys = (value_order(xf).astype(np.uint64) << np.uint64(32)) | (np.uint64(0xFFFFFFFE) - idx)[None, :]
    order = np.argsort(keys, axis=1)[:, ::-1]   # keys of a row are distinct
    rows = np.arange(xf.shape[0])
    ids = order[:, 0].astype(np.int64)
    top = order[:, :num_logprobs].astype(np.int64)
    return ids, y[rows, ids], top, y[rows[:, None], top]
