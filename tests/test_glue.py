"""The vLLM glue: quantization config, linear / lm_head methods, the CUSTOM
attention backend, DeterministicRMSNorm, plugin registration, and the KV-cache
write the backend uses.

vLLM is not installed in this image, so these tests import the glue against
tests/vllm_stub, a minimal stand-in for the vLLM API names the glue touches
(the reference's own tests need a real vLLM for this layer). CPU tests check
registration and layer selection; GPU tests check that each glue path gives
exactly the bits of the op it wraps. The KV-cache write is checked bit for bit
against a torch CPU scatter.
"""

from __future__ import annotations

import importlib
import importlib.util
import pathlib
import sys

import pytest
import torch

from _util import bits_equal

STUB = str(pathlib.Path(__file__).resolve().parent / "vllm_stub")
GLUE = ("fxpr_vllm.rms_norm", "fxpr_vllm.quantisation_config", "fxpr_vllm.attention_backend",
        "fxpr_vllm.monkey_patches", "fxpr_vllm.register", "fxpr_vllm.warmup")


def _forget_glue():
    for name in list(sys.modules):
        if name == "vllm" or name.startswith("vllm.") or name in GLUE:
            del sys.modules[name]


@pytest.fixture()
def vllm_stub(monkeypatch):
    """Import path with the stub vLLM; glue modules re-imported against it."""
    _forget_glue()
    monkeypatch.syspath_prepend(STUB)
    from fxpr_vllm import config

    config.reset_runtime_config()
    yield
    _forget_glue()
    config.reset_runtime_config()


@pytest.fixture()
def no_vllm():
    _forget_glue()
    yield
    _forget_glue()


# ---------------------------------------------------------------------------
# CPU: class wiring and registration


def test_rms_norm_without_vllm_binds_every_forward(no_vllm):
    pytest.importorskip("torch")
    if importlib.util.find_spec("vllm") is not None:
        pytest.skip("a real vLLM is importable")
    from fxpr_vllm.rms_norm import DeterministicRMSNorm, _StandaloneRMSNorm

    assert issubclass(DeterministicRMSNorm, _StandaloneRMSNorm)
    f = DeterministicRMSNorm._forward_fxp
    assert DeterministicRMSNorm.forward_cuda is f
    assert DeterministicRMSNorm.forward_hip is f
    assert DeterministicRMSNorm.forward_native is f
    layer = DeterministicRMSNorm(64, eps=1e-5)
    assert layer.variance_epsilon == 1e-5 and layer.weight.shape == (64,)


def test_rms_norm_with_vllm_overrides_rocm_dispatch(vllm_stub):
    from vllm.model_executor.layers.layernorm import RMSNorm

    from fxpr_vllm.rms_norm import DeterministicRMSNorm

    assert issubclass(DeterministicRMSNorm, RMSNorm)
    # the stub dispatches forward -> forward_hip, as vLLM's CustomOp does on ROCm
    for name in ("forward_cuda", "forward_hip", "forward_native"):
        assert getattr(DeterministicRMSNorm, name) is DeterministicRMSNorm._forward_fxp


def test_register_registers_everything_once(vllm_stub):
    from vllm.model_executor.custom_op import op_registry, op_registry_oot
    from vllm.model_executor.layers.quantization import QUANTIZATION_METHODS
    from vllm.v1.attention.backends.registry import REGISTERED, AttentionBackendEnum

    import vllm.model_executor.layers.layernorm as layernorm_mod
    from fxpr_vllm import register as reg

    reg.reset_registration()
    reg.register()
    from fxpr_vllm.quantisation_config import FixedPointConfig
    from fxpr_vllm.rms_norm import DeterministicRMSNorm

    assert QUANTIZATION_METHODS["fixedpoint"] is FixedPointConfig
    assert REGISTERED[AttentionBackendEnum.CUSTOM] == "fxpr_vllm.attention_backend.DeterministicAttentionBackend"
    assert op_registry["rms_norm"] is DeterministicRMSNorm
    assert op_registry_oot["RMSNorm"] is DeterministicRMSNorm
    assert layernorm_mod.RMSNorm is DeterministicRMSNorm
    QUANTIZATION_METHODS.clear()
    reg.register()  # idempotent
    assert not QUANTIZATION_METHODS


def test_register_respects_disable_rms_norm(vllm_stub, monkeypatch):
    monkeypatch.setenv("FXPR_DISABLE_RMS_NORM", "1")
    from fxpr_vllm import config

    config.reset_runtime_config()
    from vllm.model_executor.custom_op import op_registry

    from fxpr_vllm import register as reg

    op_registry.clear()
    reg.reset_registration()
    reg.register()
    assert "rms_norm" not in op_registry


def test_backend_path_resolves_and_early_imports_are_named(vllm_stub, caplog):
    import importlib
    import logging
    import types

    import vllm.model_executor.layers.layernorm as layernorm_mod
    from fxpr_vllm import monkey_patches

    module, _, cls = monkey_patches.BACKEND_CLASS_PATH.rpartition(".")
    from fxpr_vllm.attention_backend import DeterministicAttentionBackend

    assert getattr(importlib.import_module(module), cls) is DeterministicAttentionBackend
    # a model module that bound vLLM's RMSNorm before the hook keeps it and is named
    early = types.ModuleType("vllm.model_executor.models.early_model")
    early.RMSNorm = layernorm_mod.RMSNorm
    sys.modules[early.__name__] = early
    try:
        with caplog.at_level(logging.WARNING, logger="fxpr_vllm"):
            replaced = monkey_patches.install_rms_norm()
        assert replaced is early.RMSNorm
        assert any("early_model" in r.message for r in caplog.records)
    finally:
        del sys.modules[early.__name__]


def test_register_retries_a_failed_step(vllm_stub, monkeypatch):
    from vllm.model_executor.layers.quantization import QUANTIZATION_METHODS

    from fxpr_vllm import monkey_patches
    from fxpr_vllm import register as reg

    reg.reset_registration()
    calls = []

    def flaky():
        calls.append(1)
        if len(calls) == 1:
            raise RuntimeError("transient")
        return monkey_patches.BACKEND_CLASS_PATH

    monkeypatch.setattr(monkey_patches, "install_attention_backend", flaky)
    with pytest.raises(RuntimeError):
        reg.register()
    assert "fixedpoint" in QUANTIZATION_METHODS   # the step before the failure stays done
    QUANTIZATION_METHODS.clear()
    reg.register()
    assert len(calls) == 2 and not QUANTIZATION_METHODS


@pytest.mark.parametrize("lm_head", [True, False])
def test_quant_method_selection(vllm_stub, monkeypatch, lm_head):
    if not lm_head:
        monkeypatch.setenv("FXPR_DISABLE_LM_HEAD", "1")
    from fxpr_vllm import config

    config.reset_runtime_config()
    from vllm.model_executor.layers.linear import LinearBase
    from vllm.model_executor.layers.vocab_parallel_embedding import ParallelLMHead

    from fxpr_vllm.quantisation_config import (FixedPointConfig, FixedPointEmbeddingMethod,
                                               FixedPointLinearMethod)

    cfg = FixedPointConfig.from_config({})
    assert FixedPointConfig.get_name() == "fixedpoint"
    assert isinstance(cfg.get_quant_method(LinearBase.__new__(LinearBase), ""), FixedPointLinearMethod)
    m = cfg.get_quant_method(ParallelLMHead.__new__(ParallelLMHead), "lm_head")
    assert isinstance(m, FixedPointEmbeddingMethod) if lm_head else m is None
    assert cfg.get_quant_method(torch.nn.Linear(2, 2), "") is None


def test_attention_backend_static_interface(vllm_stub):
    from vllm.v1.attention.backend import AttentionType
    from vllm.v1.attention.backends.triton_attn import TritonAttentionMetadata

    from fxpr_vllm.attention_backend import DeterministicAttentionBackend as B
    from fxpr_vllm.attention_backend import DeterministicAttentionImpl

    assert B.get_name() == "CUSTOM"
    assert B.get_kv_cache_shape(10, 16, 8, 128) == (10, 2, 16, 8, 128)
    with pytest.raises(ValueError):
        B.get_kv_cache_shape(10, 8, 8, 128)
    assert B.get_kv_cache_stride_order() == (0, 1, 2, 3, 4)
    assert B.get_impl_cls() is DeterministicAttentionImpl
    assert B.get_metadata_cls() is TritonAttentionMetadata
    assert B.supports_head_size(128) and not B.supports_head_size(16)
    with pytest.raises(NotImplementedError):
        DeterministicAttentionImpl(8, 64, 0.125, 8, None, None, attn_type=AttentionType.ENCODER)
    with pytest.raises(NotImplementedError):
        DeterministicAttentionImpl(8, 64, 0.125, 8, None, None, kv_cache_dtype="fp8")
    impl = DeterministicAttentionImpl(8, 64, 0.125, 2, [0.5] * 8, 256, logits_soft_cap=30.0)
    assert impl.window_size == 256 and impl.logits_soft_cap == 30.0
    assert torch.allclose(impl.alibi_slopes, torch.full((8,), 0.5 * 1.4426950408889634))


# ---------------------------------------------------------------------------
# GPU: each glue path gives the bits of the op it wraps


def _bf16(*shape, seed=0, scale=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.gpu
def test_rms_norm_layer_matches_op(vllm_stub):
    from fxpr_vllm.rms_norm import DeterministicRMSNorm

    layer = DeterministicRMSNorm(512, eps=1e-6, dtype=torch.bfloat16).cuda()
    layer.weight.data.copy_(_bf16(512, seed=1, scale=0.1) + 1)
    x, r = _bf16(33, 512, seed=2).cuda(), _bf16(33, 512, seed=3).cuda()
    assert bits_equal(layer(x), torch.ops.fxpr.rms_norm_fxp(x, layer.weight, 1e-6))
    r1, r2 = r.clone(), r.clone()
    out, res = layer(x, r1)
    ref = torch.ops.fxpr.rms_norm_fxp_residual(x, r2, layer.weight, 1e-6)
    assert res is r1 and bits_equal(out, ref) and bits_equal(r1, r2)


@pytest.mark.gpu
def test_linear_method_matches_gemm_and_keeps_one_copy(vllm_stub):
    from vllm.model_executor.layers.linear import LinearBase

    from fxpr_vllm.quantisation_config import FixedPointConfig

    layer = LinearBase(256, 384, bias=True, quant_config=FixedPointConfig()).cuda()
    w = _bf16(384, 256, seed=4, scale=0.05)
    layer.weight.weight_loader(layer.weight, w.cuda())
    layer.bias.data.copy_(_bf16(384, seed=5, scale=0.1))
    storage = layer.weight.data.untyped_storage().data_ptr()
    layer.quant_method.process_weights_after_loading(layer)
    assert layer.weight is None
    assert layer.weight_native.shape == (256, 384) and layer.weight_native.stride() == (1, 256)
    assert layer.weight_native.untyped_storage().data_ptr() == storage  # a view, no copy
    for m in (1, 7, 300):
        x = _bf16(m, 256, seed=10 + m).cuda()
        ref = torch.ops.fxpr.gemm_fxp(x, w.cuda().t().contiguous(), layer.bias, 32, 16)
        assert bits_equal(layer(x), ref)


@pytest.mark.gpu
def test_lm_head_method_logits_and_lookup(vllm_stub):
    from vllm.model_executor.layers.vocab_parallel_embedding import ParallelLMHead

    from fxpr_vllm.quantisation_config import FixedPointConfig

    head = ParallelLMHead(1000, 128, quant_config=FixedPointConfig()).cuda()
    w = _bf16(1000, 128, seed=6, scale=0.02).cuda()
    head.weight.data.copy_(w)
    head.quant_method.process_weights_after_loading(head)
    x = _bf16(5, 128, seed=7).cuda()
    logits = head.quant_method.apply(head, x)
    assert bits_equal(logits, torch.ops.fxpr.gemm_fxp(x, w.t().contiguous(), None, 32, 16))
    ids = torch.tensor([0, 999, 17], device="cuda")
    assert bits_equal(head(ids), w[ids])


def _cache_scatter_cpu(key, value, kv, slots):
    kv = kv.clone()
    nb, _, bs = kv.shape[:3]
    for t, s in enumerate(slots.tolist()):
        if 0 <= s < nb * bs:
            kv[s // bs, 0, s % bs] = key[t]
            kv[s // bs, 1, s % bs] = value[t]
    return kv


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_reshape_and_cache_bit_exact(dtype):
    import fxpr_vllm  # noqa: F401

    g = torch.Generator("cpu").manual_seed(8)
    T, H, D, NB, BS = 37, 4, 64, 9, 16
    qkv = torch.randn(T, (8 + 2 * H) * D, generator=g).to(dtype)
    key = qkv[:, 8 * D:(8 + H) * D].view(T, H, D)           # strided views, as split from qkv
    value = qkv[:, (8 + H) * D:].view(T, H, D)
    slots = torch.randperm(NB * BS, generator=g)[:T].to(torch.int64)
    slots[3] = -1                      # padding token
    slots[5] = NB * BS + 100           # out of range: skipped
    kv = torch.randn(NB, 2, BS, H, D, generator=g).to(dtype)
    ref = _cache_scatter_cpu(key, value, kv, slots)
    kv_d = kv.cuda()
    torch.ops.fxpr.reshape_and_cache(key.cuda(), value.cuda(), kv_d, slots.cuda())
    assert bits_equal(kv_d, ref)
    # int32 slot mappings are accepted too
    kv_d2 = kv.cuda()
    torch.ops.fxpr.reshape_and_cache(key.cuda(), value.cuda(), kv_d2, slots.to(torch.int32).cuda())
    assert bits_equal(kv_d2, ref)


@pytest.mark.gpu
def test_attention_impl_matches_ops(vllm_stub):
    from vllm.v1.attention.backends.triton_attn import TritonAttentionMetadata

    from fxpr_vllm.attention_backend import DeterministicAttentionImpl

    Hq, Hkv, D, BS, NB = 8, 2, 64, 16, 32
    impl = DeterministicAttentionImpl(Hq, D, D ** -0.5, Hkv, None, None)
    g = torch.Generator("cpu").manual_seed(9)
    # two requests: a prefill of 20 tokens (no context) and a decode token with 40 of context
    q_lens, ctx = [20, 1], [0, 40]
    T = sum(q_lens)
    kv = torch.zeros(NB, 2, BS, Hkv, D, dtype=torch.bfloat16, device="cuda")
    bt = torch.randperm(NB, generator=g)[:8].view(2, 4).to(torch.int32)
    # history of request 1 already cached
    hist_k = torch.randn(40, Hkv, D, generator=g).to(torch.bfloat16)
    hist_v = torch.randn(40, Hkv, D, generator=g).to(torch.bfloat16)
    hist_slots = torch.tensor([int(bt[1, p // BS]) * BS + p % BS for p in range(40)])
    torch.ops.fxpr.reshape_and_cache(hist_k.cuda(), hist_v.cuda(), kv, hist_slots.cuda())
    slots = torch.tensor([int(bt[0, p // BS]) * BS + p % BS for p in range(20)] +
                         [int(bt[1, 40 // BS]) * BS + 40 % BS])
    q = torch.randn(T, Hq * D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(T, Hkv * D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(T, Hkv * D, generator=g).to(torch.bfloat16).cuda()
    qsl = torch.tensor([0, 20, 21], dtype=torch.int32, device="cuda")
    sl = torch.tensor([20, 41], dtype=torch.int32, device="cuda")
    meta = TritonAttentionMetadata(T, 20, qsl, 41, sl, bt.cuda(), slots.cuda())
    kv_ref = kv.clone()
    impl.do_kv_cache_update(None, k, v, kv, meta.slot_mapping)
    torch.ops.fxpr.reshape_and_cache(k.view(T, Hkv, D), v.view(T, Hkv, D), kv_ref, meta.slot_mapping)
    assert bits_equal(kv, kv_ref)
    out_buf = torch.empty(T, Hq * D, dtype=torch.bfloat16, device="cuda")
    out = impl.forward(None, q, k, v, kv, meta, output=out_buf)
    ref = torch.empty(T, Hq, D, dtype=torch.bfloat16, device="cuda")
    torch.ops.fxpr.unified_attention_fxp(q.view(T, Hq, D), kv, ref, qsl, sl, meta.block_table, 20, None,
                                         True, D ** -0.5, 32, 16, 0.0, 0, 0)
    assert out.data_ptr() == out_buf.data_ptr()
    assert bits_equal(out.view(T, Hq, D), ref)
    # profiling call without metadata: zeros
    assert torch.count_nonzero(impl.forward(None, q, k, v, kv, None)) == 0


@pytest.mark.gpu
def test_warmups_run_clean_once(caplog):
    # the warm-ups swallow errors by design, so a broken launch would only
    # show as a logged warning: require none, and a second call to do nothing
    import logging

    import fxpr_vllm  # noqa: F401
    from fxpr_vllm import warmup

    warmup._done.clear()
    dev = torch.device("cuda")
    w = _bf16(512, 384, seed=11, scale=0.05).cuda().t()
    with caplog.at_level(logging.WARNING, logger="fxpr_vllm"):
        for dtype in (torch.bfloat16, torch.float16):
            warmup.warmup_attention(8, 2, 128, dtype, dev, 0, 0.0, 32, 16)
        warmup.warmup_rms_norm(4096, torch.bfloat16, dev)
        warmup.warmup_gemm(w, 32, 16)
        warmup.warmup_gemm(w, 64, 16)
    assert not [r for r in caplog.records if "warm-up" in r.message], caplog.text
    n = len(warmup._done)
    assert n == 5
    warmup.warmup_gemm(w, 32, 16)
    warmup.warmup_rms_norm(4096, torch.bfloat16, dev)
    assert len(warmup._done) == n
