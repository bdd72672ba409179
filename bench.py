#!/usr/bin/env python
"""Benchmark of the fxpr fixed-point kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workloads a,b,...]

Prints ONE JSON line. The headline (`metric`/`value`) is BASELINE.json's
metric: the fixed-point lm_head GEMM in TFLOP/s (bf16 A[8192,4096] x
B[4096,128256], Q16.16 in int32) whose `roofline` is against the dense bf16
MFMA peak; the paged split-K decode attention (HBM GB/s and % of roofline),
RMSNorm+residual and log-softmax lines ride along under `extra`, each with
its own roofline. A step is one call of the workload's op on one batch of
seeded synthetic input already resident in HBM; each workload times exactly K
steps between HIP events recorded on the stream the kernels run on, after W
warmup steps, with a device synchronize on both sides. Inputs whose total
footprint would fit in the 256 MB MALL are rotated across copies so the
figures are HBM figures.

`cpu_baseline` times the numpy oracle (oracle/, the CPU restatement of the
same fixed-point arithmetic) on a bounded sample of the headline workload on
this box's host cores.
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
    """HBM bytes per launch of the workload's dominant kernel, from the
    rocprofv3 FETCH_SIZE / WRITE_SIZE counter runs summarised in
    profiles/hbm_traffic.md (counter KiB scaled by the factor a plain copy of
    known size reads), or None when the workload was not profiled."""
    path = ROOT / "profiles" / "hbm_traffic.md"
    try:
        for line in path.read_text().splitlines():
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 5 and cells[0] == f"`{workload}`":
                return int(cells[-1].replace(",", ""))
    except (OSError, ValueError):
        pass
    return None


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
           "splits": KG.resolve_split_k(M, N, K, dtype, split_k),
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
    "decode_attn": lambda s, w: wl_decode(s, w, 0),
    "decode_attn_s1": lambda s, w: wl_decode(s, w, 1),
    "decode_attn_s2": lambda s, w: wl_decode(s, w, 2),
    "decode_attn_s4": lambda s, w: wl_decode(s, w, 4),
    "decode_attn_s8": lambda s, w: wl_decode(s, w, 8),
    "decode_attn_s16": lambda s, w: wl_decode(s, w, 16),
    "prefill_attn": lambda s, w: wl_prefill(s, w),
    "gemm_lm_head": lambda s, w: wl_gemm(s, w, 8192),
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
    "hbm_copy": lambda s, w: wl_hbm_copy(s, w),
}
HEADLINE_ORDER = ["gemm_lm_head", "decode_attn", "rms_norm"]


# ---------------------------------------------------------------------------
# CPU baseline: the numpy oracle on a bounded sample of the headline workload


def cpu_baseline(headline: str, budget_s: float) -> dict:
    import numpy as np

    from oracle import rows as OR

    threads = 1  # numpy elementwise arithmetic runs on one core
    if headline.startswith("gemm"):
        from oracle import gemm as OG

        try:
            from threadpoolctl import threadpool_info

            threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
        except Exception:  # noqa: BLE001
            threads = os.cpu_count() or 1
        M, K, Nn = 64, 4096, 2048
        rng = np.random.default_rng(0)
        a = (rng.standard_normal((M, K)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        b = ((rng.standard_normal((K, Nn)) * 0.02).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        reps, t0 = 0, time.perf_counter()
        while True:
            OG.gemm(a, b, None, "bf16", 32, 16)
            reps += 1
            if time.perf_counter() - t0 > budget_s:
                break
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(2.0 * M * K * Nn / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
                "kind": "port",
                "sample": f"oracle.gemm.gemm bf16 A[{M},{K}] x B[{K},{Nn}] Q16/i32 (numpy, BLAS "
                          f"float64 tile dots), {reps} reps in {budget_s:.0f}s"}
    if headline.startswith("rms_norm"):
        H = 4096
        rows = 64
        rng = np.random.default_rng(0)
        x = (rng.standard_normal((rows, H)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        r = (rng.standard_normal((rows, H)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        w = np.full(H, 0x3F80, np.uint16)
        reps, t0 = 0, time.perf_counter()
        while True:
            OR.rms_norm(x, w, 1e-6, "bf16", residual=r)
            reps += 1
            if time.perf_counter() - t0 > budget_s:
                break
        dt = (time.perf_counter() - t0) / reps
        gbs = 4 * rows * H * 2 / dt / 1e9
        return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"oracle.rows.rms_norm bf16 [{rows},{H}] + residual, "
                          f"{reps} reps in {budget_s:.0f}s"}
    raise ValueError(headline)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workloads", default="all")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
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
        results[name]["roofline"]["traffic"] = measured_traffic(name)
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
        "extra": {k: v for k, v in results.items() if k != headline},
        "host": {"cpu_count": os.cpu_count(), "cpu_model": cpu_model(),
                 "torch_threads": torch.get_num_threads(),
                 "gpu": torch.cuda.get_device_name(0)},
    }
    if not args.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(headline, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
