"""Every op under HIP graph capture (torch.cuda.CUDAGraph).

vLLM serves decode steps from captured graphs (the reference defers its
warm-up while a capture is running, fxpr_vllm/warmup.py:38-40, 119-120), so
each op must be capturable: no host synchronisation, no device allocation
outside the caching allocator, no memset nodes. Each test captures one call,
then replays it several times; before every replay new inputs are copied into
the captured input tensors and the outputs are poisoned, the program's own
eager work and a synchronisation run between replays, and every replay must
equal an eager call on the same inputs bit for bit. The last test captures
the first launch of every kernel family in a fresh process (the large-tile
kernels set their LDS size attribute on first use).
"""

from __future__ import annotations

import os
import subprocess
import sys
import textwrap

import pytest
import torch

import fxpr_vllm  # noqa: F401
from tests._util import bits_equal

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPLAYS = 3


def _randn(shape, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(DEV)


def _poison(t: torch.Tensor) -> None:
    if t.is_floating_point():
        t.fill_(float("nan"))
    else:
        t.fill_(-7)


def check_capture(make_inputs, run):
    """make_inputs(seed) -> dict of input tensors; run(inputs) -> output
    tensor or tuple (an input the op writes in place is returned as an
    output; copying the next inputs in restores it before each replay)."""
    static = make_inputs(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):          # settle the allocator outside capture
        run({k: v.clone() for k, v in static.items()})
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run(static)
    outs = outs if isinstance(outs, tuple) else (outs,)
    for rep in range(REPLAYS):
        fresh = make_inputs(rep + 1)
        eager = run({k: v.clone() for k, v in fresh.items()})
        eager = eager if isinstance(eager, tuple) else (eager,)
        for o in outs:
            _poison(o)
        for k, v in fresh.items():
            static[k].copy_(v)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert bits_equal(o, e), f"replay {rep}, output {i}"
    graph.reset()


@pytest.mark.parametrize("M", [1, 32, 256])
@pytest.mark.parametrize("bits", [32, 64])
def test_capture_gemm(M, bits):
    K, N = 1024, 2048
    w = _randn((N, K), 1, scale=0.02)

    def make(seed):
        return {"a": _randn((M, K), 10 + seed), "bias": _randn((N,), 20 + seed)}

    check_capture(make, lambda t: torch.ops.fxpr.gemm_fxp(t["a"], w.t(), t["bias"], bits, 16))


def test_capture_gemm_split_k():
    from fxpr_vllm._kernels import gemm as KG

    K, N, M = 4096, 1024, 64
    w = _randn((N, K), 2, scale=0.02)
    check_capture(lambda s: {"a": _randn((M, K), 30 + s)},
                  lambda t: KG.gemm_fxp_run(t["a"], w.t(), None, 32, 16, split_k=4))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_capture_rms_norm(dtype):
    H = 4096

    def make(seed):
        return {"x": _randn((48, H), 40 + seed, dtype, scale=3.0),
                "w": _randn((H,), 50 + seed, dtype, scale=0.1) + 1}

    check_capture(make, lambda t: torch.ops.fxpr.rms_norm_fxp(t["x"], t["w"], 1e-6))


def test_capture_rms_norm_residual():
    H = 4096

    def make(seed):
        return {"x": _randn((48, H), 60 + seed), "r": _randn((48, H), 70 + seed),
                "w": _randn((H,), 80 + seed, scale=0.1) + 1}

    def run(t):
        y = torch.ops.fxpr.rms_norm_fxp_residual(t["x"], t["r"], t["w"], 1e-6)
        return y, t["r"]

    check_capture(make, run)


@pytest.mark.parametrize("bits,frac", [(32, 16), (64, 32)])
def test_capture_log_softmax(bits, frac):
    check_capture(lambda s: {"x": _randn((8, 128256), 90 + s, scale=4.0)},
                  lambda t: torch.ops.fxpr.log_softmax_fxp(t["x"], bits, frac))


def test_capture_casts_and_row_sum():
    def run(t):
        q = torch.ops.fxpr.float_to_fixed(t["x"], 32, 16)
        s = torch.ops.fxpr.fixed_row_sum(q, 64)
        return q, s, torch.ops.fxpr.fixed_to_float(s, 32, 16)

    check_capture(lambda s: {"x": _randn((64, 1000), 100 + s, torch.float32, scale=50.0)}, run)


def test_capture_reshape_and_cache():
    T, H, D, NB, BS = 40, 8, 128, 16, 16
    slots = torch.randperm(NB * BS, generator=torch.Generator("cpu").manual_seed(5))[:T].to(DEV)

    def make(seed):
        return {"k": _randn((T, H, D), 110 + seed), "v": _randn((T, H, D), 120 + seed),
                "kv": _randn((NB, 2, BS, H, D), 130 + seed)}

    def run(t):
        torch.ops.fxpr.reshape_and_cache(t["k"], t["v"], t["kv"], slots)
        return t["kv"]

    check_capture(make, run)


def _paged(q_lens, ctx, hq=32, hkv=8, d=128, ps=16, seed=0):
    g = torch.Generator("cpu").manual_seed(seed)
    sls = [c + q for c, q in zip(ctx, q_lens)]
    maxb = max(-(-s // ps) for s in sls)
    nb = len(sls) * maxb + 5
    bt = torch.randperm(nb, generator=g)[: len(sls) * maxb].to(torch.int32).reshape(len(sls), maxb)
    starts = [0]
    for n in q_lens:
        starts.append(starts[-1] + n)
    meta = (torch.tensor(starts, dtype=torch.int32, device=DEV), torch.tensor(sls, dtype=torch.int32, device=DEV),
            bt.to(DEV))
    return meta, (starts[-1], hq, d), (nb, 2, ps, hkv, d)


@pytest.mark.parametrize("q_lens,ctx,splits", [
    ([1] * 16, [3000 + 97 * i for i in range(16)], 0),     # decode, automatic split count
    ([1] * 16, [3000 + 97 * i for i in range(16)], 16),    # decode, 16 splits (workspace in the graph pool)
    ([1, 200, 1, 7], [5000, 300, 64, 900], 0),            # mixed prefill + decode
])
def test_capture_attention(q_lens, ctx, splits):
    (qsl, sl, bt), qshape, kvshape = _paged(q_lens, ctx)
    maxq = max(q_lens)

    def make(seed):
        return {"q": _randn(qshape, 140 + seed), "kv": _randn(kvshape, 150 + seed)}

    def run(t):
        o = torch.empty_like(t["q"])
        torch.ops.fxpr.unified_attention_fxp(t["q"], t["kv"], o, qsl, sl, bt, maxq, None, True, None, 32, 16,
                                             0.0, 0, splits)
        return o

    check_capture(make, run)


_FIRST_LAUNCH = textwrap.dedent("""
    import sys, torch
    sys.path[:0] = {paths!r}
    import fxpr_vllm  # noqa: F401
    dev = "cuda"
    g = torch.Generator("cpu").manual_seed(0)
    a = torch.randn(512, 1024, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(768, 1024, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    x = torch.randn(16, 4096, generator=g).to(torch.bfloat16).to(dev)
    lw = torch.ones(4096, dtype=torch.bfloat16, device=dev)
    q = torch.randn(300, 8, 128, generator=g).to(torch.bfloat16).to(dev)
    kv = torch.randn(40, 2, 16, 2, 128, generator=g).to(torch.bfloat16).to(dev)
    qsl = torch.tensor([0, 299, 300], dtype=torch.int32, device=dev)
    sl = torch.tensor([299, 320], dtype=torch.int32, device=dev)
    bt = torch.arange(40, dtype=torch.int32, device=dev).reshape(2, 20)

    def step():
        c = torch.ops.fxpr.gemm_fxp(a, w.t(), None, 32, 16)
        c64 = torch.ops.fxpr.gemm_fxp(a, w.t(), None, 64, 16)
        y = torch.ops.fxpr.rms_norm_fxp(x, lw, 1e-6)
        o = torch.empty_like(q)
        torch.ops.fxpr.unified_attention_fxp(q, kv, o, qsl, sl, bt, 299, None, True, None, 32, 16, 0.0, 0, 1)
        o2 = torch.empty_like(q)
        torch.ops.fxpr.unified_attention_fxp(q, kv, o2, qsl, sl, bt, 299, None, True, None, 32, 16, 0.0, 0, 4)
        return c, c64, y, o, o2

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):          # the first launch of every kernel is inside the capture
        outs = step()
    graph.replay()
    torch.cuda.synchronize()
    eager = step()
    torch.cuda.synchronize()
    for i, (o, e) in enumerate(zip(outs, eager)):
        assert torch.equal(o.view(torch.int16), e.view(torch.int16)), i
    print("first-launch capture ok", flush=True)
""")


def test_first_launch_inside_capture_fresh_process(tmp_path):
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    paths = [os.path.join(root, "vllm-triton-fixed-point-reductions_amd"), root]
    script = tmp_path / "first_launch.py"
    script.write_text(_FIRST_LAUNCH.format(paths=paths))
    res = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "first-launch capture ok" in res.stdout


def test_capture_sample_greedy():
    check_capture(lambda s: {"x": _randn((16, 128256), 160 + s, scale=4.0)},
                  lambda t: torch.ops.fxpr.sample_greedy_fxp(t["x"], 20, 32, 16))
