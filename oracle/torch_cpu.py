"""The oracle's fixed-point GEMM, RMSNorm, log-softmax, casts and decode
attention as PyTorch CPU code (multi-threaded), for the benchmark's CPU
baseline.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). The same arithmetic as
oracle.gemm / oracle.rows / oracle.numerics / oracle.attention, step for step: fp32 values
held in torch.float32 (one IEEE rounding per operation), float64 tile dots
rounded once to fp32, integers in int64; tests/test_oracle_torch_cpu.py pins
every function bit for bit against the numpy restatement. Storage
conventions follow the numpy oracle's: 'bf16' arrays are uint16 bit patterns
(passed here as int16 or int32 tensors holding them).
"""

from __future__ import annotations

import torch

from .numerics import EXP2_C, EXP_FLOOR, LN2_HI, LN2_LO, LOG2E, LOG_C, SQRT2

F32, F64, I64 = torch.float32, torch.float64, torch.int64


def load(a: torch.Tensor, io: str) -> torch.Tensor:
    if io == "bf16":
        return (a.to(torch.int32) & 0xFFFF).bitwise_left_shift(16).view(F32)
    return a.to(F32)


def store(f: torch.Tensor, io: str) -> torch.Tensor:
    """fp32 -> storage of the I/O type (RNE; bf16 NaN -> 0x7FC0, as
    oracle.numerics.f32_to_bf16 and the kernels)."""
    if io == "bf16":
        u = f.to(F32).view(torch.int32).to(I64) & 0xFFFFFFFF
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
        return torch.where(torch.isnan(f), torch.full_like(r, 0x7FC0), r).to(torch.int32)
    return f.to({"f16": torch.float16, "f32": F32, "f64": F64}[io])


def ldexp32(x: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """fl32(x * 2^k) with one rounding for any integer k (the product is exact
    in float64, the conversion rounds once, subnormals included)."""
    return (x.to(F64) * torch.pow(2.0, k.to(F64))).to(F32)


def rne_sat(s: torch.Tensor, int_bits: int) -> torch.Tensor:
    """RNE then saturate to int_bits, NaN -> 0 (oracle.numerics.rne_sat)."""
    r = torch.round(s.to(F64))          # round half to even, exact for fp32 inputs
    r = torch.where(torch.isnan(r), torch.zeros_like(r), r)
    hi = 2.0 ** (int_bits - 1)
    over, under = r >= hi, r <= -hi
    q = torch.where(over | under, torch.zeros_like(r), r).to(I64)
    q = torch.where(over, torch.full_like(q, (1 << (int_bits - 1)) - 1), q)
    return torch.where(under, torch.full_like(q, -(1 << (int_bits - 1))), q)


def float_to_fixed(x: torch.Tensor, int_bits: int, frac_bits: int) -> torch.Tensor:
    return rne_sat(x.to(F32) * (2.0 ** frac_bits), int_bits)


def fixed_row_sum(q: torch.Tensor, int_bits: int) -> torch.Tensor:
    """Exact sum (int64 inputs may not wrap: callers keep |sum| < 2^63), one saturation."""
    hi = (1 << (int_bits - 1)) - 1
    return q.to(I64).sum(-1).clamp(-hi - 1, hi)


def fixed_to_f32(q: torch.Tensor, frac_bits: int) -> torch.Tensor:
    return q.to(F32) * torch.tensor(2.0 ** -frac_bits, dtype=F32)


def gemm(a, b, bias, io: str, int_bits: int, frac_bits: int, block_k: int | None = None) -> torch.Tensor:
    """oracle.gemm.gemm: per K-tile float64 dot rounded to fp32, RNE_sat(P * 2^f)
    summed in int64 and wrapped to int_bits, epilogue in fp32."""
    af, bf = load(a, io).to(F64), load(b, io).to(F64)
    M, K = af.shape
    N = bf.shape[1]
    bk = block_k or (64 if io == "f32" else 128)
    scale = torch.tensor(2.0 ** frac_bits, dtype=F32)
    acc = torch.zeros(M, N, dtype=I64)
    for t in range(0, K, bk):
        p = (af[:, t:t + bk] @ bf[t:t + bk, :]).to(F32)
        acc += rne_sat(p * scale, int_bits)
    if int_bits < 64:
        m, h = 1 << int_bits, 1 << (int_bits - 1)
        acc = torch.remainder(acc + h, m) - h
    c = fixed_to_f32(acc, frac_bits)
    if bias is not None:
        c = c + load(bias, io if bias.dtype != F32 else "f32").reshape(1, N)
    return store(c, io)


RMS_SUM_FRAC = 40


def rms_norm(x, w, eps: float, io: str, residual=None):
    """oracle.rows.rms_norm: the per-row block floating-point integer sum."""
    H = x.shape[-1]
    xf = load(x, io).reshape(-1, H)
    wf = load(w, io).reshape(H)
    if residual is not None:
        v = xf + load(residual, io).reshape(-1, H)
        new_r = store(v, io)
        u = load(new_r, io)
    else:
        v, new_r, u = xf, None, xf
    mbits = (v.view(torch.int32) & 0x7FFFFFFF).amax(-1)
    e = torch.clamp(mbits >> 23, min=1) - 127
    finite = mbits < 0x7F800000
    s = ldexp32(v, (-e)[:, None])
    t = torch.where(finite[:, None], s * s, torch.zeros_like(s))
    q = torch.round(t.to(F64) * 2.0 ** RMS_SUM_FRAC).to(I64)
    total = q.sum(-1)                   # < 2^63 for H <= 2^21
    mean_scaled = total.to(F32) / torch.tensor(float(H), dtype=F32)
    ms = ldexp32(mean_scaled, 2 * e - RMS_SUM_FRAC)
    ms = torch.where(finite, ms, mbits.view(F32))
    rrms = torch.tensor(1.0, dtype=F32) / torch.sqrt(ms + torch.tensor(eps, dtype=F32))
    y = store((u * wf[None, :]) * rrms[:, None], io).reshape(x.shape)
    return y, (None if new_r is None else new_r.reshape(x.shape))


def _fma_f32(a, b, c):
    """fl32(a * b + c), one rounding (oracle.numerics.fma_f32 in torch)."""
    a64, b64, c64 = a.to(F64), b.to(F64), c.to(F64)
    p = a64 * b64
    s = p + c64
    bv = s - p
    err = (p - (s - bv)) + (c64 - bv)
    r = s.to(F32)
    r64 = r.to(F64)
    up = torch.nextafter(r, torch.full_like(r, float("inf"))).to(F64)
    dn = torch.nextafter(r, torch.full_like(r, float("-inf"))).to(F64)
    tie_up = (s == (r64 + up) * 0.5) & (err > 0)
    tie_dn = (s == (r64 + dn) * 0.5) & (err < 0)
    fin = torch.isfinite(s) & torch.isfinite(err)
    return torch.where(fin & tie_up, up, torch.where(fin & tie_dn, dn, r64)).to(F32)


def exp_scaled(d: torch.Tensor, frac_bits: int) -> torch.Tensor:
    ok = d >= float(EXP_FLOOR)
    dd = torch.where(ok, d, torch.zeros_like(d))
    tt = dd * float(LOG2E)
    k = torch.round(tt)
    r = tt - k
    p = torch.full_like(r, float(EXP2_C[7]))
    for coef in EXP2_C[6::-1]:
        p = _fma_f32(p, r, torch.full_like(r, float(coef)))
    out = ldexp32(p, k + frac_bits)
    return torch.where(ok, out, torch.zeros_like(out))


def log_own(y: torch.Tensor) -> torch.Tensor:
    bits = y.view(torch.int32)
    e = (bits >> 23) - 127
    m = ((bits & 0x007FFFFF) | 0x3F800000).view(F32)
    big = m > float(SQRT2)
    m = torch.where(big, m * 0.5, m)
    e = torch.where(big, e + 1, e)
    one = torch.tensor(1.0, dtype=F32)
    s = (m - one) / (m + one)
    z = s * s
    p = torch.full_like(z, float(LOG_C[4]))
    for coef in LOG_C[3::-1]:
        p = p * z + float(coef)
    lnm = (s * 2.0) * p
    fe = e.to(F32)
    return fe * float(LN2_HI) + (fe * float(LN2_LO) + lnm)


def log_softmax(x, io_in: str, io_out: str, int_bits: int, frac_bits: int) -> torch.Tensor:
    """oracle.rows.log_softmax (sums kept below 2^63 by the callers' sizes)."""
    V = x.shape[-1]
    xf = load(x, io_in).reshape(-1, V)
    m = xf.amax(-1)
    m = torch.where(torch.isnan(xf).any(-1), torch.full_like(m, float("nan")), m)
    e = exp_scaled(xf - m[:, None], frac_bits)
    total = rne_sat(e, int_bits).sum(-1)
    S = total.to(F32) * torch.tensor(2.0 ** -frac_bits, dtype=F32)
    lnS = torch.where(total == 0, torch.full_like(S, float("-inf")),
                      log_own(torch.where(total == 0, torch.ones_like(S), S)))
    lse = m + lnS
    return store(xf - lse[:, None], io_out).reshape(x.shape)


def _wrap(v: torch.Tensor, int_bits: int) -> torch.Tensor:
    if int_bits == 64:
        return v
    m, h = 1 << int_bits, 1 << (int_bits - 1)
    return torch.remainder(v + h, m) - h


def _rescale(x: torch.Tensor, f: torch.Tensor, int_bits: int) -> torch.Tensor:
    """oracle.attention._rescale: RNE(fl64(x) * fl64(f)), saturated."""
    r = torch.round(_wrap(x, int_bits).to(F64) * f.to(F64))
    lim = 2.0 ** (int_bits - 1)
    r = torch.where(r >= lim, torch.full_like(r, lim - 1), torch.where(r < -lim, torch.full_like(r, -lim), r))
    return r.to(I64)


def decode_attention(q, kv_cache, seq_lens, block_table, io: str, softmax_scale: float,
                     int_bits: int, frac_bits: int, chunk_keys: int = 512) -> torch.Tensor:
    """oracle.attention.unified_attention(chunk_keys=512) for decode batches:
    one query per request (query_start_loc = arange(R + 1)), causal, no
    window, softcap or ALiBi, all heads of a request at once. q [R, Hq, D];
    kv_cache [NB, 2, page, Hkv, D]; returns o [R, Hq, D] in storage form."""
    qf = load(q, io).to(F64)
    kv = load(kv_cache, io)
    R, Hq, D = qf.shape
    _, _, ps, Hkv, _ = kv.shape
    G = Hq // Hkv
    bn = 32 if io == "f32" else 64
    ss_log2 = torch.tensor(float(softmax_scale) * 1.4426950408889634, dtype=F32)
    scale = torch.tensor(2.0 ** frac_bits, dtype=F32)
    out = torch.zeros(R, Hq, D, dtype=F32)
    for r in range(R):
        L = int(seq_lens[r])
        nblk = -(-L // ps)
        blocks = block_table[r, :nblk].long()
        K = kv[blocks, 0].reshape(nblk * ps, Hkv, D)[:L].to(F64)
        Lp = -(-L // bn) * bn
        V = torch.zeros(Lp, Hkv, D, dtype=F64)
        V[:L] = kv[blocks, 1].reshape(nblk * ps, Hkv, D)[:L]
        qh = qf[r].reshape(Hkv, G, D)
        s = torch.full((Hkv, G, Lp), float("-inf"), dtype=F32)
        s[:, :, :L] = torch.matmul(qh, K.permute(1, 2, 0)).to(F32) * ss_log2
        M = torch.full((Hkv, G), float("-inf"), dtype=F32)
        Dn = torch.zeros(Hkv, G, dtype=I64)
        W = torch.zeros(Hkv, G, D, dtype=I64)
        for k0 in range(0, Lp, chunk_keys):
            k1 = min(Lp, k0 + chunk_keys)
            sc = s[:, :, k0:k1]
            m_raw = sc.amax(-1)
            m = torch.where(torch.isfinite(m_raw), m_raw, torch.zeros_like(m_raw))
            w = (sc - m[..., None]).to(F64).exp2().to(F32)
            den = _wrap(rne_sat(w * scale, int_bits).sum(-1), int_bits)
            p = load(store(w, io), io).to(F64)
            nt = (k1 - k0) // bn
            pv = torch.matmul(p.reshape(Hkv, G, nt, bn).permute(0, 2, 1, 3),
                              V[k0:k1].reshape(nt, bn, Hkv, D).permute(2, 0, 1, 3)).to(F32)
            wv = _wrap(rne_sat(pv * scale, int_bits).sum(1), int_bits)
            # merge_chunk: fold the chunk into the running state
            live = torch.isfinite(m_raw)
            Mn = torch.where(live, torch.maximum(M, m_raw), M)
            fa = torch.where(live, (M - Mn).to(F64).exp2(), torch.ones_like(M, dtype=F64)).to(F32)
            fb = torch.where(live, (m_raw - Mn).to(F64).exp2(), torch.zeros_like(M, dtype=F64)).to(F32)
            fa = torch.where(torch.isnan(fa), torch.zeros_like(fa), fa)
            fb = torch.where(torch.isnan(fb), torch.zeros_like(fb), fb)
            Dnn = _wrap(_rescale(Dn, fa, int_bits) + _rescale(den, fb, int_bits), int_bits)
            Wn = _wrap(_rescale(W, fa[..., None], int_bits) + _rescale(wv, fb[..., None], int_bits), int_bits)
            M = torch.where(live, Mn, M)
            Dn = torch.where(live, Dnn, Dn)
            W = torch.where(live[..., None], Wn, W)
        den_f = torch.maximum(fixed_to_f32(Dn, frac_bits), torch.tensor(1e-6, dtype=F32))
        out[r] = (fixed_to_f32(W, frac_bits) / den_f[..., None]).reshape(Hq, D)
    return store(out, io)
