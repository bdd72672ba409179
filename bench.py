#!/usr/bin/env python
"""Benchmark of the fxpr fixed-point kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workloads a,b,...]

Prints ONE JSON line. The headline (`metric`/`value`) is BASELINE.json's
metric: the fixed-point lm_head GEMM in TFLOP/s (bf16 A[8192,4096] x
B[4096,128256], Q16.16 in int32) whose `roofline` is against the dense bf16
MFMA peak. The metric's second half, the paged split-K decode attention in
HBM GB/s, is `decode` (automatic splits and each forced count). Every other
BASELINE configuration rides along under `workloads` with its own roofline:
the other GEMM shapes, RMSNorm + residual and log-softmax (HBM), causal
prefill attention (MFMA), config 1's cast / row-sum / RMSNorm chain, and
config 5's Llama-3-8B-shaped decoder (tokens/s at batch 32 / 8 / 1, report
only). A step is one call of the workload's op on one batch of
seeded synthetic input already resident in HBM; each workload times exactly K
steps between HIP events recorded on the stream the kernels run on, after W
warmup steps, with a device synchronize on both sides. Inputs whose total
footprint would fit in the 256 MB MALL are rotated across copies so the
figures are HBM figures.

`cpu_baseline` is the CPU emulation of the headline's fixed-point path
(oracle/torch_cpu.py, PyTorch on every host thread, pinned bit for bit to the
numpy oracle) timed on this box's host cores on a column slice of the
headline shape, extrapolated and labelled; `cpu_suite` holds the same
emulation timed per BASELINE configuration (configs 1, 2a, 4 and GEMM
M <= 32 whole, the rest on labelled samples), with the thread count of each.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
PKG_ROOT = ROOT / "vllm-triton-fixed-point-reductions_amd"
for _p in (str(PKG_ROOT), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
FP32_PEAK_TFLOPS = 157.3
MALL_BYTES = 256 << 20

METRIC = "fxp lm_head GEMM TFLOP/s; paged decode attn HBM GB/s (% of roofline)"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# Untimed settling (seconds) after the warmup steps: set by main() for every
# workload but the headline (which keeps exactly --warmup steps and runs
# first in the default order). A short kernel timed right after another
# workload's long run (the 9 ms GEMM steps) otherwise runs before the clocks
# have recovered: decode attention measured 7 % slower first in line than in
# the same run's later identical configuration.
_SETTLE_S = 0.0


def time_op(fn, inputs, steps: int, warmup: int) -> float:
    """Average ms per call over `steps` calls, rotating through `inputs`."""
    import torch

    for i in range(warmup):
        fn(*inputs[i % len(inputs)])
    torch.cuda.synchronize()
    t0, i = time.perf_counter(), warmup
    while time.perf_counter() - t0 < _SETTLE_S:
        for _ in range(max(1, warmup)):
            fn(*inputs[i % len(inputs)])
            i += 1
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(*inputs[i % len(inputs)])
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def copies_for(bytes_per_set: int) -> int:
    """Input sets to rotate so one pass over them exceeds 2x the MALL."""
    return max(1, min(8, -(-2 * MALL_BYTES // max(1, bytes_per_set))))


def hbm_roofline(bytes_per_call: float, ms: float) -> dict:
    gbs = bytes_per_call / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}


def measured_traffic(workload: str):
    """(HBM bytes per launch of the workload's dominant kernel, where that
    figure comes from): the rocprofv3 FETCH_SIZE / WRITE_SIZE counter runs
    summarised in profiles/hbm_traffic.md (counter KiB scaled by the factor a
    plain copy of known size reads), stamped with the commit of the kernels
    it measured; (None, None) when the workload was not profiled. A counter
    run cannot share the process it measures, so the figure is not re-taken
    here."""
    path = ROOT / "profiles" / "hbm_traffic.md"
    try:
        text = path.read_text()
        stamp = next((ln.split(":", 1)[1].strip() for ln in text.splitlines()
                      if ln.lower().startswith("kernels measured at commit")), "unknown commit")
        for line in text.splitlines():
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 5 and cells[0] == f"`{workload}`":
                return int(cells[-1].replace(",", "")), f"profiles/hbm_traffic.md ({stamp})"
    except (OSError, ValueError):
        pass
    return None, None


def mfma_roofline(flops: float, ms: float, peak: float = BF16_PEAK_TFLOPS) -> dict:
    tf = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(tf / peak, 4), "traffic": None}


# ---------------------------------------------------------------------------
# workloads (each returns a dict; the synthetic data follows BASELINE.json)


def wl_rms_norm(steps, warmup, T=16384, H=4096):
    import torch

    from fxpr_vllm._kernels import rows as K

    g = torch.Generator("cpu").manual_seed(0)
    dev = "cuda"
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    r0 = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(H, generator=g) * 0.1 + 1.0).to(torch.bfloat16).to(dev)
    nbytes = 4 * T * H * 2 + 2 * H
    sets = [(x, r0.clone(), w) for _ in range(copies_for(nbytes))]

    def fn(xx, rr, ww):
        return K.rms_norm_fxp_residual_run(xx, rr, ww, 1e-6)

    ms = time_op(fn, sets, steps, warmup)
    return {"workload": f"rms_norm_residual bf16 [{T},{H}]",
            "ms": round(ms, 5), "bytes": nbytes, "roofline": hbm_roofline(nbytes, ms)}


def _logits(R, V, seed=0):
    import torch

    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(R, V, generator=g) * 4.0
    mask = torch.rand(R, V, generator=g) < 0.01
    sign = torch.where(torch.rand(R, V, generator=g) < 0.5, -1.0, 1.0)
    return torch.where(mask, 30.0 * sign, x).to(torch.bfloat16)


def wl_log_softmax(steps, warmup, int_bits=32, frac_bits=16, fp32_out=False, R=256, V=128256):
    import torch

    x = _logits(R, V).to("cuda")
    out_dtype = torch.float32 if fp32_out else None
    nbytes = R * V * (2 + (4 if fp32_out else 2))
    sets = [(x.clone(),) for _ in range(copies_for(nbytes))]

    def fn(xx):
        return torch.ops.fxpr.log_softmax_fxp(xx, int_bits, frac_bits, out_dtype)

    ms = time_op(fn, sets, steps, warmup)
    return {"workload": f"log_softmax bf16 [{R},{V}] -> {'f32' if fp32_out else 'bf16'} "
                        f"Q{frac_bits}/i{int_bits}",
            "ms": round(ms, 5), "bytes": nbytes, "roofline": hbm_roofline(nbytes, ms)}


_WEIGHTS: dict = {}


def _weight(N, K, dtype, std, seed):
    """[N, K] row-major weight (vLLM's layout), seeded on the CPU, cached."""
    import torch

    key = (N, K, dtype, std, seed)
    if key not in _WEIGHTS:
        g = torch.Generator("cpu").manual_seed(seed)
        w = torch.empty(N, K, dtype=dtype)
        step = 8192
        for i in range(0, N, step):  # bounded host memory
            w[i:i + step] = (torch.randn(min(step, N - i), K, generator=g) * std).to(dtype)
        _WEIGHTS.clear()
        _WEIGHTS[key] = w.to("cuda")
    return _WEIGHTS[key]


def wl_gemm(steps, warmup, M, N=128256, K=4096, dtype_name="bf16", int_bits=32, frac_bits=16,
            split_k=0):
    """lm_head / linear GEMM. B = W^T with W [N, K] row-major: the K-contiguous
    layout the fixed-point linear method keeps (no transposed copy)."""
    import torch

    from fxpr_vllm._kernels import gemm as KG

    dtype = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype_name]
    esz = torch.tensor([], dtype=dtype).element_size()
    w = _weight(N, K, dtype, 0.02, seed=1)
    g = torch.Generator("cpu").manual_seed(2)
    b_bytes = N * K * esz
    a = torch.randn(M, K, generator=g).to(dtype).to("cuda")
    sets = [(a, w.t())]
    if b_bytes * 2 < 2 * MALL_BYTES:  # weights that fit in the MALL: rotate copies
        sets += [(a, w.clone().t()) for _ in range(copies_for(b_bytes) - 1)]

    def fn(aa, bb):
        return KG.gemm_fxp_run(aa, bb, None, int_bits, frac_bits, split_k=split_k)

    ms = time_op(fn, sets, steps, warmup)
    flops = 2.0 * M * N * K
    nbytes = esz * (M * K + K * N + M * N)
    peak = FP32_PEAK_TFLOPS if dtype == torch.float32 else BF16_PEAK_TFLOPS
    res = {"workload": f"gemm_fxp {dtype_name} A[{M},{K}] x B[{K},{N}] (B K-contiguous) "
                       f"Q{frac_bits}/i{int_bits}",
           "ms": round(ms, 5), "flops": flops, "bytes": nbytes,
           "splits": KG.resolve_split_k(M, N, K, dtype, int_bits, split_k),
           "mfma": mfma_roofline(flops, ms, peak), "hbm": hbm_roofline(nbytes, ms)}
    # the bounding roofline: HBM for skinny M, MFMA from the ridge point on
    res["roofline"] = res["mfma"] if flops / nbytes > peak * 1e12 / (HBM_PEAK_GBS * 1e9) else res["hbm"]
    return res


def wl_decode(steps, warmup, splits=0, int_bits=32, frac_bits=16, B=64, hq=32, hkv=8, d=128, ps=16,
              pool=1 << 16, seed=0):
    """Paged split-K decode attention: 64 one-token requests, contexts
    U[512, 8192], 16-token pages in a 2^16-page pool (BASELINE.json's fourth
    configuration). Context lengths,
    the block table (consecutive slices of a permutation of the pool) and q
    come from a seeded CPU generator; the 4 GiB KV pool from a seeded device
    generator (generating it on the host would dominate the run)."""
    import torch

    g = torch.Generator("cpu").manual_seed(seed)
    sl = torch.randint(512, 8193, (B,), generator=g, dtype=torch.int32)
    maxb = 8192 // ps
    bt = torch.randperm(pool, generator=g).to(torch.int32)[: B * maxb].reshape(B, maxb)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16).to("cuda")
    key = ("kvpool", pool, ps, hkv, d)
    if key not in _WEIGHTS:
        _WEIGHTS.clear()
        gd = torch.Generator("cuda").manual_seed(seed + 1)
        _WEIGHTS[key] = torch.randn(pool, 2, ps, hkv, d, generator=gd, device="cuda", dtype=torch.bfloat16)
    kv = _WEIGHTS[key]
    qsl = torch.arange(B + 1, dtype=torch.int32, device="cuda")
    sl_d, bt_d = sl.to("cuda"), bt.to("cuda")
    o = torch.empty_like(q)
    scale = 1.0 / d ** 0.5

    def fn():
        torch.ops.fxpr.unified_attention_fxp(q, kv, o, qsl, sl_d, bt_d, 1, None, True, scale,
                                             int_bits, frac_bits, 0.0, 0, splits)

    ms = time_op(fn, [()], steps, warmup)
    sum_l = int(sl.sum())
    nbytes = sum_l * hkv * d * 2 * 2 + 2 * (B * hq * d * 2) + sum(-(-int(x) // ps) for x in sl) * 4 + 2 * B * 4
    from fxpr_vllm._kernels import attention as KA

    s_eff = KA.pick_num_splits(splits, B, hkv, hq // hkv, 1, maxb, ps)
    return {"workload": f"decode attn bf16 B={B} Hq={hq} Hkv={hkv} d={d} ctx~U[512,8192] "
                        f"(sum {sum_l}) page {ps} splits={s_eff} Q{frac_bits}/i{int_bits}",
            "ms": round(ms, 5), "bytes": nbytes, "splits": s_eff, "roofline": hbm_roofline(nbytes, ms)}


def wl_prefill(steps, warmup, splits=0, int_bits=32, frac_bits=16, B=4, L=2048, hq=32, hkv=8, d=128, ps=16,
               seed=0):
    """Paged causal prefill attention: B prompts of L new tokens each (no
    cached context), Llama-3-8B head shape, bf16, pages of one shuffled pool.
    Algorithmic flops = 4 * Hq * D * sum over rows of the keys it attends
    (QK^T and PV, 2 flops per multiply-add), against the bf16 MFMA peak."""
    import torch

    g = torch.Generator("cpu").manual_seed(seed)
    nb = B * (L // ps)
    bt = torch.randperm(nb, generator=g).to(torch.int32).reshape(B, L // ps)
    q = torch.randn(B * L, hq, d, generator=g).to(torch.bfloat16).to("cuda")
    kv = torch.randn(nb, 2, ps, hkv, d, generator=g).to(torch.bfloat16).to("cuda")
    qsl = (torch.arange(B + 1, dtype=torch.int32) * L).to("cuda")
    sl = torch.full((B,), L, dtype=torch.int32, device="cuda")
    bt_d = bt.to("cuda")
    o = torch.empty_like(q)
    scale = 1.0 / d ** 0.5

    def fn():
        torch.ops.fxpr.unified_attention_fxp(q, kv, o, qsl, sl, bt_d, L, None, True, scale,
                                             int_bits, frac_bits, 0.0, 0, splits)

    ms = time_op(fn, [()], steps, warmup)
    flops = 4 * hq * d * B * (L * (L + 1) // 2)
    return {"workload": f"prefill attn bf16 causal B={B} L={L} Hq={hq} Hkv={hkv} d={d} page {ps} "
                        f"Q{frac_bits}/i{int_bits}",
            "ms": round(ms, 5), "flops": flops, "roofline": mfma_roofline(flops, ms, BF16_PEAK_TFLOPS)}


def wl_config1(steps, warmup, int_bits=32):
    """BASELINE config 1 on the GPU: fp32 x [4096, 4096] ~N(0,1) through
    float_to_fixed -> fixed_row_sum -> fixed_to_float (Q16.16 in int32 or
    int64), then RMSNorm and RMSNorm + residual (weight ~N(1, 0.1), eps 1e-6),
    one step = the five launches. Algorithmic bytes: the cast reads 4 n and
    writes b/8 n, the row sum reads b/8 n, RMSNorm moves 8 n, RMSNorm +
    residual 16 n (n = 4096^2; the [4096] results are negligible)."""
    import torch

    n = 4096
    g = torch.Generator("cpu").manual_seed(0)
    x = torch.randn(n, n, generator=g).to("cuda")
    r0 = torch.randn(n, n, generator=g).to("cuda")
    w = (torch.randn(n, generator=g) * 0.1 + 1.0).to("cuda")
    nb = int_bits // 8
    nbytes = n * n * (4 + nb + nb + 8 + 16)
    sets = [(x, r0.clone(), w) for _ in range(copies_for(nbytes))]

    def fn(xx, rr, ww):
        q = torch.ops.fxpr.float_to_fixed(xx, int_bits, 16)
        torch.ops.fxpr.fixed_to_float(torch.ops.fxpr.fixed_row_sum(q, int_bits), 32, 16)
        torch.ops.fxpr.rms_norm_fxp(xx, ww, 1e-6)
        torch.ops.fxpr.rms_norm_fxp_residual(xx, rr, ww, 1e-6)

    ms = time_op(fn, sets, steps, warmup)
    return {"workload": f"config 1: fp32 [{n},{n}] cast -> row sum -> cast (Q16.16 in int{int_bits}), "
                        f"RMSNorm, RMSNorm + residual",
            "ms": round(ms, 5), "bytes": nbytes, "roofline": hbm_roofline(nbytes, ms)}


def wl_e2e_llama(batches=(32, 8, 1), prompt=2048, max_new=128):
    """BASELINE config 5 on the library's own harness (tests/e2e_decoder.py):
    a random-init Llama-3-8B-shaped decoder (32 layers, hidden 4096, 32/8
    heads of 128, FFN 14336, vocab 128256, bf16 weights ~N(0, 0.02); merged
    q/k/v and gate/up projections as vLLM holds them) built only from the
    fxpr ops, served as vLLM serves it: `batch` random-token prompts of
    `prompt` tokens prefilled in one eager step, one eager decode step, then
    the remaining decode steps of the whole batch replayed from a captured
    HIP graph (greedy sampler with top-5 log-probabilities), `max_new` new
    tokens per request in all, at each batch size. Reported per batch size:
    decode tokens/s over the replayed steps (a step = one token for every
    request) and the prefill's tokens/s."""
    import torch

    sys.path.insert(0, str(ROOT / "tests"))
    from e2e_decoder import Config, Decoder, run_graph

    pages = max(batches) * -(-(prompt + max_new) // 16) + 8
    model = Decoder(Config.llama3_8b(pages), seed=0)
    g = torch.Generator("cpu").manual_seed(5)
    prompts = [torch.randint(0, 128256, (prompt,), generator=g).tolist() for _ in range(max(batches))]
    per = {}
    for b in batches:
        t = {}
        run_graph(model, prompts[:b], max_new, timing=t)
        ms = t["decode_s"] * 1e3 / t["decode_steps"]
        per[f"batch{b}"] = {"decode_ms_per_step": round(ms, 4),
                            "decode_tokens_per_s": round(b * t["decode_steps"] / t["decode_s"], 1),
                            "prefill_tokens_per_s": round(b * prompt / t["prefill_s"], 1)}
        log(f"  config 5 batch {b}: {per[f'batch{b}']}")
    del model
    torch.cuda.empty_cache()
    head = per[f"batch{max(batches)}"]
    return {"workload": f"config 5: Llama-3-8B-shaped decoder on the fxpr ops, prompts {prompt}, greedy "
                        f"{max_new} new tokens (top-5 log-probs), decode from a captured HIP graph, "
                        f"batch {'/'.join(str(b) for b in batches)}",
            "ms": head["decode_ms_per_step"], "per_batch": per,
            "roofline": {"bound": "mixed", "achieved": head["decode_tokens_per_s"], "peak": None,
                         "unit": "tokens/s", "frac": None, "traffic": None}}


def wl_hbm_copy(steps, warmup, nbytes=1 << 30):
    """torch copy_ of a known size: the reference point for HBM bandwidth and
    for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    src = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    ms = time_op(lambda: dst.copy_(src), [()], steps, warmup)
    return {"workload": f"torch copy_ {nbytes} B", "ms": round(ms, 5), "bytes": 2 * nbytes,
            "roofline": hbm_roofline(2 * nbytes, ms)}


WORKLOADS = {
    "gemm_lm_head": lambda s, w: wl_gemm(s, w, 8192),
    "decode_attn": lambda s, w: wl_decode(s, w, 0),
    "decode_attn_s1": lambda s, w: wl_decode(s, w, 1),
    "decode_attn_s2": lambda s, w: wl_decode(s, w, 2),
    "decode_attn_s4": lambda s, w: wl_decode(s, w, 4),
    "decode_attn_s8": lambda s, w: wl_decode(s, w, 8),
    "decode_attn_s16": lambda s, w: wl_decode(s, w, 16),
    "prefill_attn": lambda s, w: wl_prefill(s, w),
    "gemm_lm_head_m2048": lambda s, w: wl_gemm(s, w, 2048),
    "gemm_lm_head_m256": lambda s, w: wl_gemm(s, w, 256),
    "gemm_lm_head_m32": lambda s, w: wl_gemm(s, w, 32),
    "gemm_lm_head_m1": lambda s, w: wl_gemm(s, w, 1),
    "gemm_lm_head_m8192_i64": lambda s, w: wl_gemm(s, w, 8192, int_bits=64),
    "gemm_f16_14336_m8192": lambda s, w: wl_gemm(s, w, 8192, N=14336, dtype_name="f16"),
    "gemm_f32_14336_m8192": lambda s, w: wl_gemm(max(3, s // 4), 1, 8192, N=14336, dtype_name="f32"),
    "rms_norm": lambda s, w: wl_rms_norm(s, w),
    "log_softmax": lambda s, w: wl_log_softmax(s, w, 32, 16),
    "log_softmax_f32out_q32i64": lambda s, w: wl_log_softmax(s, w, 64, 32, fp32_out=True),
    "config1_q16_i32": lambda s, w: wl_config1(s, w, 32),
    "config1_q16_i64": lambda s, w: wl_config1(s, w, 64),
    "e2e_llama3_8b": lambda s, w: wl_e2e_llama(),
    "hbm_copy": lambda s, w: wl_hbm_copy(s, w),
}
HEADLINE_ORDER = ["gemm_lm_head", "decode_attn", "rms_norm"]


# ---------------------------------------------------------------------------
# CPU baseline: the CPU emulation of the same fixed-point path, timed per
# BASELINE configuration on this box's host cores. GEMM, RMSNorm,
# log-softmax, the casts and the decode attention run as PyTorch CPU code on
# every host thread (oracle/torch_cpu.py, pinned bit for bit to the numpy
# oracle). Shapes too slow to run whole are timed on a documented sample and
# extrapolated linearly in the sampled dimension; each entry says which.


def _timed(fn, min_s: float = 0.0):
    """(seconds per call, calls): at least one call, repeated up to min_s."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        if time.perf_counter() - t0 >= min_s:
            return (time.perf_counter() - t0) / n, n


def cpu_suite(scale: float = 1.0) -> dict:
    """Per-configuration CPU timings. `scale` multiplies the sample sizes of
    the extrapolated entries (1.0: about a minute in all)."""
    import torch

    from oracle import torch_cpu as TC

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    torch.randn(1 << 20).sum()   # start the thread pool outside the timed calls
    g = torch.Generator("cpu").manual_seed(0)
    out = {}

    def randn(*shape, std=1.0, mean=0.0):
        return torch.randn(*shape, generator=g) * std + mean

    def bf16(t):
        return TC.store(t, "bf16")

    def entry(value, unit, seconds, cores, sample, extrapolated=False, impl="torch_cpu"):
        return {"value": round(value, 6), "unit": unit, "seconds_full_shape": round(seconds, 4), "cores": cores,
                "kind": "port", "impl": impl, "sample": sample, "extrapolated": extrapolated}

    # config 1: fp32 [4096, 4096] cast -> row sum -> cast; RMSNorm + residual
    n = 4096
    x, r, w = randn(n, n), randn(n, n), randn(n, std=0.1, mean=1.0)
    for bits in (32, 64):
        dt, _ = _timed(lambda: TC.fixed_to_f32(TC.fixed_row_sum(TC.float_to_fixed(x, bits, 16), bits), 16))
        nbytes = 4 * n * n + (bits // 8) * n * n * 2
        out[f"config1_cast_rowsum_q16_i{bits}"] = entry(nbytes / dt / 1e9, "GB/s", dt, threads,
                                                         f"full [{n},{n}] fp32, Q16.16 in int{bits}")
    dt, _ = _timed(lambda: TC.rms_norm(x, w, 1e-6, "f32", residual=r))
    out["config1_rms_norm_residual_f32"] = entry(16 * n * n / dt / 1e9, "GB/s", dt, threads, f"full [{n},{n}] fp32")

    # config 2a: RMSNorm + residual, bf16 [16384, 4096]
    T, H = 16384, 4096
    xb, rb, wb = bf16(randn(T, H)), bf16(randn(T, H)), bf16(randn(H, std=0.1, mean=1.0))
    dt, _ = _timed(lambda: TC.rms_norm(xb, wb, 1e-6, "bf16", residual=rb))
    out["config2a_rms_norm_residual_bf16"] = entry(4 * T * H * 2 / dt / 1e9, "GB/s", dt, threads,
                                                   f"full [{T},{H}] bf16")
    del xb, rb

    # config 2b: log-softmax, bf16 [256, 128256] ~N(0,4) with 1 % at +-30
    R, V = 256, 128256
    rs = max(8, int(64 * scale))
    lg = randn(rs, V, std=4.0)
    lg = torch.where(torch.rand(rs, V, generator=g) < 0.01, torch.full_like(lg, 30.0), lg)
    lgb = bf16(lg)
    for bits, frac in ((32, 16), (64, 32)):
        dt, _ = _timed(lambda: TC.log_softmax(lgb, "bf16", "bf16", bits, frac))
        full = dt * R / rs
        out[f"config2b_log_softmax_q{frac}_i{bits}"] = entry(R * V * 4 / full / 1e9, "GB/s", full, threads,
                                                              f"{rs} of {R} rows x {V}, bf16 in and out",
                                                              rs != R)

    # config 3: lm_head GEMM, bf16 A[M, 4096] x B[4096, 128256]; M <= 32 whole,
    # larger M on a column slice of B (time linear in N)
    K, N = 4096, 128256
    wfull = bf16(randn(K, N, std=0.02))
    for M in (1, 32, 256, 2048, 8192):
        ncols = N if M <= 32 else max(128, int({256: 16384, 2048: 2048, 8192: 512}[M] * scale))
        a = bf16(randn(M, K))
        bsl = wfull if ncols == N else wfull[:, :ncols].contiguous()
        dt, _ = _timed(lambda: TC.gemm(a, bsl, None, "bf16", 32, 16))
        full = dt * N / ncols
        out[f"config3_gemm_bf16_m{M}"] = entry(2.0 * M * K * N / full / 1e12, "TFLOP/s", full, threads,
                                               f"A[{M},{K}] x B[{K},{ncols}] of N={N}, Q16.16 in int32",
                                               ncols != N)
    del wfull
    # config 3': f16 / fp32 A[8192, 4096] x B[4096, 14336] on a column slice
    for io in ("f16", "f32"):
        M, N2 = 8192, 14336
        nc = max(128, int(512 * scale))
        a = TC.store(randn(M, K), io)
        bsl = TC.store(randn(K, nc, std=0.02), io)
        dt, _ = _timed(lambda: TC.gemm(a, bsl, None, io, 32, 16))
        full = dt * N2 / nc
        out[f"config3p_gemm_{io}_m{M}"] = entry(2.0 * M * K * N2 / full / 1e12, "TFLOP/s", full, threads,
                                                f"A[{M},{K}] x B[{K},{nc}] of N={N2}, Q16.16 in int32", True)

    # config 4: decode attention, 64 one-token requests with the GPU bench's
    # seeded context lengths U[512, 8192], 16-token pages, whole (the chunked
    # algorithm as PyTorch CPU code on every host thread)
    gl = torch.Generator("cpu").manual_seed(0)
    sl = torch.randint(512, 8193, (64,), generator=gl, dtype=torch.int32)
    nbk = [-(-int(L) // 16) for L in sl]
    kv = bf16(randn(sum(nbk), 2, 16, 8, 128))
    bt = torch.zeros(64, max(nbk), dtype=torch.int32)
    off = 0
    for i, nb in enumerate(nbk):
        bt[i, :nb] = torch.arange(off, off + nb, dtype=torch.int32)
        off += nb
    q = bf16(randn(64, 32, 128))
    dt, _ = _timed(lambda: TC.decode_attention(q, kv, sl, bt, "bf16", 128 ** -0.5, 32, 16))
    nbytes = int(sl.sum()) * 4096 + 2 * 64 * 32 * 128 * 2
    out["config4_decode_attention"] = entry(nbytes / dt / 1e9, "GB/s", dt, threads,
                                            f"full: 64 requests, sum of contexts {int(sl.sum())}, Q16.16/i32")
    return out


def cpu_baseline_from(suite: dict, headline: str) -> dict:
    key = {"gemm_lm_head": "config3_gemm_bf16_m8192", "decode_attn": "config4_decode_attention",
           "rms_norm": "config2a_rms_norm_residual_bf16"}[headline]
    e = dict(suite[key])
    e["config"] = key
    return e


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workloads", default="all")
    ap.add_argument("--cpu-scale", type=float, default=1.0,
                    help="sample size factor of the extrapolated CPU baseline entries")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(requested --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import fxpr_vllm  # noqa: F401

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)

    names = list(WORKLOADS) if args.workloads == "all" else args.workloads.split(",")
    results = {}
    global _SETTLE_S
    headline = next((h for h in HEADLINE_ORDER if h in names), names[0])
    for name in names:
        log(f"workload {name} ...")
        _SETTLE_S = 0.0 if name == headline else 0.2  # the headline: exactly W warmup steps
        results[name] = WORKLOADS[name](args.steps, args.warmup)
        traffic, source = measured_traffic(name)
        results[name]["roofline"]["traffic"] = traffic
        if traffic is not None:
            results[name]["roofline"]["traffic_source"] = source
        log(f"  {json.dumps(results[name])}")

    _WEIGHTS.clear()
    head = results[headline]
    rf = head["roofline"]
    value = rf["achieved"]
    out = {
        "metric": METRIC,
        "value": value,
        "unit": rf["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 MFMA, int32 fixed-point accumulate" if headline.startswith("gemm")
                 else "bf16 in, int32 fixed-point accumulate",
        "data": "synthetic (seeded torch CPU generator, copied to HBM)",
        "config": {"workload": head["workload"], "headline": headline},
        "roofline": rf,
    }
    # the metric's second half: paged split-K decode attention (HBM)
    dec = {k: v for k, v in results.items() if k.startswith("decode_attn")}
    if dec:
        out["decode"] = {("auto" if k == "decode_attn" else k.split("_")[-1]): compact(v) for k, v in dec.items()}
    if not args.no_cpu:
        log("cpu baseline (oracle per configuration) ...")
        suite = cpu_suite(args.cpu_scale)
        out["cpu_baseline"] = cpu_baseline_from(suite, headline)
        out["cpu_suite"] = {k: {kk: v[kk] for kk in ("value", "unit", "cores", "sample", "extrapolated")}
                            for k, v in suite.items()}
        log(f"  {json.dumps(suite)}")
    out["workloads"] = {k: compact(v) for k, v in results.items() if k != headline}
    out["host"] = {"cpu_count": os.cpu_count(), "cpu_model": cpu_model(),
                   "torch_threads": torch.get_num_threads(), "gpu": torch.cuda.get_device_name(0)}
    print(json.dumps(out), flush=True)


def compact(r: dict) -> dict:
    """A workload's result for the JSON line: what ran, ms per step and its
    roofline (achieved, unit, fraction of peak, measured HBM traffic)."""
    rf = r["roofline"]
    c = {"workload": r["workload"], "ms": r["ms"], "achieved": rf["achieved"], "unit": rf["unit"],
         "frac": rf["frac"], "bound": rf["bound"]}
    if rf.get("traffic") is not None:
        c["traffic"] = rf["traffic"]
    for k in ("splits", "per_batch"):
        if k in r:
            c[k] = r[k]
    return c


if __name__ == "__main__":
    main()
