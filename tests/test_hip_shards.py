"""GPU parity of the shard halves for more than one device (the integer
exchanges a multi-device layout needs, shown on one GPU):

* a row-parallel (K-sharded) GEMM: each K-shard's integer accumulators
  (gemm_fxp_partial), summed across shards with integer adds (what an
  all-reduce SUM on int32 / int64 does, in any order), then gemm_fxp's
  epilogue (gemm_fxp_finish), equal gemm_fxp on the whole K bit for bit;
* a vocab-parallel log-softmax: the MAX of the shards' row maxima, the
  integer SUM of the shards' exact row sums against it, then each shard's
  outputs, equal log_softmax_fxp on the whole rows bit for bit.

The last test runs the exchange for real: two processes on the one GPU, each
holding one K-shard and one vocab shard, exchange through torch.distributed
(gloo, host tensors) and check the unsharded bits.
"""

from __future__ import annotations

import os
import socket
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest
import torch

import fxpr_vllm  # noqa: F401
from tests._util import mismatch_report, nan_aware_equal

pytestmark = pytest.mark.gpu
DEV = "cuda"


def wrap_sum(parts, int_bits):
    """Integer SUM of shard accumulators, wrapping as the accumulator type."""
    total = torch.stack([p.to(torch.int64) for p in parts]).sum(0)
    if int_bits == 64:
        return total
    return (torch.remainder(total + (1 << 31), 1 << 32) - (1 << 31)).to(torch.int32)


def sharded_gemm(a, b, bias, bits, frac, cuts):
    parts = [torch.ops.fxpr.gemm_fxp_partial(a[:, k0:k1].contiguous(), b[k0:k1], bits, frac)
             for k0, k1 in zip(cuts[:-1], cuts[1:])]
    return torch.ops.fxpr.gemm_fxp_finish(wrap_sum(parts, bits), bias, bits, frac, a.dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M", [1, 32, 300])
@pytest.mark.parametrize("bits,frac", [(32, 16), (64, 16), (16, 8)])
def test_k_sharded_gemm_equals_gemm(dtype, M, bits, frac):
    # K = 1024 in shards of 384 / 256 / 384 columns (K-tile boundaries for
    # every input type), B the transposed view of an [N, K] weight as the
    # linear methods keep it, N ragged, with a bias
    g = torch.Generator("cpu").manual_seed(M + bits)
    K, N = 1024, 1000
    a = torch.randn(M, K, generator=g).to(dtype).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype).to(DEV)
    bias = torch.randn(N, generator=g).to(dtype).to(DEV)
    want = torch.ops.fxpr.gemm_fxp(a, w.t(), bias, bits, frac)
    for cuts in ((0, 384, 640, 1024), (0, 512, 1024), (0, 1024)):
        got = sharded_gemm(a, w.t(), bias, bits, frac, cuts)
        assert torch.equal(got.view(torch.int16) if dtype != torch.float32 else got.view(torch.int32),
                           want.view(torch.int16) if dtype != torch.float32 else want.view(torch.int32)), \
            (cuts, mismatch_report(got.cpu(), want.cpu()))


def test_k_sharded_gemm_wraps_like_the_accumulator():
    # large exact partials: a 32-bit accumulator wraps in the shards and in
    # the whole-K GEMM alike (int16: wraps at the epilogue)
    g = torch.Generator("cpu").manual_seed(3)
    a = torch.randint(-64, 65, (16, 512), generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randint(-64, 65, (512, 64), generator=g).to(torch.bfloat16).to(DEV)
    for bits, frac in ((32, 16), (16, 8)):
        want = torch.ops.fxpr.gemm_fxp(a, b, None, bits, frac)
        got = sharded_gemm(a, b, None, bits, frac, (0, 128, 256, 512))
        assert torch.equal(got, want), bits


def test_gemm_finish_from_unaligned_accumulators():
    # accumulators at a 4-byte offset (the finish takes element loads) and
    # 7 x 13 of them (not a multiple of 4)
    g = torch.Generator("cpu").manual_seed(8)
    a = torch.randn(7, 256, generator=g).to(torch.bfloat16).to(DEV)
    b = (torch.randn(256, 13, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    want = torch.ops.fxpr.gemm_fxp(a, b, None, 32, 16)
    acc = torch.ops.fxpr.gemm_fxp_partial(a, b, 32, 16)
    store = torch.zeros(acc.numel() + 1, dtype=torch.int32, device=DEV)
    shifted = store[1:].view(7, 13)
    shifted.copy_(acc)
    assert shifted.data_ptr() % 16 != 0
    assert torch.equal(torch.ops.fxpr.gemm_fxp_finish(shifted, None, 32, 16, torch.bfloat16), want)


def test_gemm_partial_errors_and_empty():
    a = torch.zeros(4, 256, dtype=torch.bfloat16, device=DEV)
    b = torch.zeros(256, 8, dtype=torch.bfloat16, device=DEV)
    acc = torch.ops.fxpr.gemm_fxp_partial(a, b, 32, 16)
    assert acc.dtype == torch.int32 and acc.shape == (4, 8) and not acc.any()
    assert torch.ops.fxpr.gemm_fxp_partial(a, b, 64, 16).dtype == torch.int64
    with pytest.raises(TypeError):
        torch.ops.fxpr.gemm_fxp_finish(acc.to(torch.int64), None, 32, 16, torch.bfloat16)
    with pytest.raises(ValueError):
        torch.ops.fxpr.gemm_fxp_partial(a, b[:128], 32, 16)
    empty = torch.ops.fxpr.gemm_fxp_partial(a[:0], b, 32, 16)
    assert empty.shape == (0, 8)


def _logits(rows, cols, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * 4.0
    mask = torch.rand(rows, cols, generator=g) < 0.01
    x = torch.where(mask, 30.0 * torch.where(torch.rand(rows, cols, generator=g) < 0.5, -1.0, 1.0), x)
    x[1] = 0.25                      # a flat row
    x[2, 5000] = 90.0                # a dominant logit
    x[3, 777] = float("nan")        # NaN row
    x[4, :] = float("-inf")          # every logit -inf
    x[4, 100] = 1.0
    return x


def sharded_log_softmax(x, bits, frac, cuts, out_dtype):
    shards = [x[:, c0:c1].contiguous() for c0, c1 in zip(cuts[:-1], cuts[1:])]
    m = torch.stack([torch.ops.fxpr.log_softmax_fxp_shard_max(s) for s in shards]).amax(0)
    total = torch.stack([torch.ops.fxpr.log_softmax_fxp_shard_sum(s, m, bits, frac) for s in shards]).sum(0)
    return torch.cat([torch.ops.fxpr.log_softmax_fxp_shard_finish(s, m, total, frac, out_dtype) for s in shards], 1)


@pytest.mark.parametrize("bits,frac", [(32, 16), (64, 32), (16, 8)])
@pytest.mark.parametrize("dtype,out_dtype", [(torch.bfloat16, None), (torch.bfloat16, torch.float32),
                                             (torch.float32, None), (torch.float16, torch.float32)])
def test_vocab_sharded_log_softmax_equals_log_softmax(bits, frac, dtype, out_dtype):
    # 128256 columns in four uneven shards (one of an odd width: element
    # loads) and in eight even ones
    x = _logits(6, 128_256, seed=bits + frac).to(dtype).to(DEV)
    want = torch.ops.fxpr.log_softmax_fxp(x, bits, frac, out_dtype)
    for cuts in ((0, 30001, 64128, 100000, 128256), tuple(range(0, 128257, 16032))):
        got = sharded_log_softmax(x, bits, frac, cuts, out_dtype)
        assert nan_aware_equal(got.cpu(), want.cpu()), (cuts, mismatch_report(got.cpu(), want.cpu()))


def test_shard_ops_validate():
    x = torch.zeros(3, 64, dtype=torch.bfloat16, device=DEV)
    m = torch.ops.fxpr.log_softmax_fxp_shard_max(x)
    assert m.dtype == torch.float32 and m.shape == (3,)
    with pytest.raises(ValueError):
        torch.ops.fxpr.log_softmax_fxp_shard_sum(x, m[:2], 32, 16)
    with pytest.raises(TypeError):
        torch.ops.fxpr.log_softmax_fxp_shard_finish(x, m, m, 16)
    with pytest.raises(ValueError):
        torch.ops.fxpr.log_softmax_fxp_shard_sum(x, m, 33, 16)


_WORKER = textwrap.dedent("""
    import os, sys
    sys.path[:0] = [os.environ["FXPR_PKG"], os.environ["FXPR_ROOT"]]
    import torch
    import torch.distributed as dist
    import fxpr_vllm
    from tests.test_hip_shards import _logits, wrap_sum
    rank, world = int(os.environ["RANK"]), int(os.environ["WORLD_SIZE"])
    dist.init_process_group("gloo", rank=rank, world_size=world)
    dev = "cuda"
    g = torch.Generator("cpu").manual_seed(11)
    a = torch.randn(32, 2048, generator=g).to(torch.bfloat16)
    w = (torch.randn(4096, 2048, generator=g) * 0.05).to(torch.bfloat16)
    x = _logits(6, 128_256, seed=5).to(torch.bfloat16)
    # rank r holds K columns [1024 r, 1024 (r + 1)) and vocab columns [64128 r, 64128 (r + 1))
    k0, c0 = 1024 * rank, 64128 * rank
    acc = torch.ops.fxpr.gemm_fxp_partial(a[:, k0:k0 + 1024].contiguous().to(dev),
                                          w[:, k0:k0 + 1024].contiguous().to(dev).t(), 32, 16)
    acc64 = acc.cpu().to(torch.int64)                 # gloo: host tensors, synchronous copies
    dist.all_reduce(acc64, op=dist.ReduceOp.SUM)
    c = torch.ops.fxpr.gemm_fxp_finish(wrap_sum([acc64], 32).to(dev), None, 32, 16, torch.bfloat16)
    xs = x[:, c0:c0 + 64128].contiguous().to(dev)
    ms = [torch.empty(6) for _ in range(world)]
    dist.all_gather(ms, torch.ops.fxpr.log_softmax_fxp_shard_max(xs).cpu())
    m = torch.stack(ms).amax(0)                      # NaN-propagating MAX
    s = torch.ops.fxpr.log_softmax_fxp_shard_sum(xs, m.to(dev), 32, 16).cpu()
    dist.all_reduce(s, op=dist.ReduceOp.SUM)
    y = torch.ops.fxpr.log_softmax_fxp_shard_finish(xs, m.to(dev), s.to(dev), 16, torch.float32).cpu()
    ys = [torch.empty_like(y) for _ in range(world)]
    dist.all_gather(ys, y)
    if rank == 0:
        want_c = torch.ops.fxpr.gemm_fxp(a.to(dev), w.to(dev).t(), None, 32, 16).cpu()
        want_y = torch.ops.fxpr.log_softmax_fxp(x.to(dev), 32, 16, torch.float32).cpu()
        got_y = torch.cat(ys, 1)
        same_y = bool(((got_y == want_y) | (got_y.isnan() & want_y.isnan())).all())
        print("GEMM_SAME", torch.equal(c.cpu(), want_c), "LSM_SAME", same_y, flush=True)
    dist.destroy_process_group()
""")


def test_two_process_exchange_over_gloo():
    root = Path(__file__).resolve().parents[1]
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    env = dict(os.environ, MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port), WORLD_SIZE="2",
               FXPR_PKG=str(root / "vllm-triton-fixed-point-reductions_amd"), FXPR_ROOT=str(root))
    procs = [subprocess.Popen([sys.executable, "-c", _WORKER], cwd=root, env=dict(env, RANK=str(r)),
                              stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True) for r in range(2)]
    outs = []
    for p in procs:
        try:
            outs.append(p.communicate(timeout=200))
        except subprocess.TimeoutExpired:
            for q in procs:
                q.kill()
            raise
    assert all(p.returncode == 0 for p in procs), [o[1][-2000:] for o in outs]
    assert "GEMM_SAME True LSM_SAME True" in outs[0][0], outs[0]
