"""The CUSTOM attention backend: vLLM attention through unified_attention_fxp.

Same backend interface and behaviour as the reference
(fxpr_vllm/attention_backend.py:40-277): decoder-only, fp16 / bf16 / fp32,
"auto" / fp16 / bf16 KV cache (no fp8, no output scales), KV cache laid out
[num_blocks, 2, block_size, num_kv_heads, head_size] with block sizes that
are multiples of 16, causal attention with the automatic KV-split policy,
ALiBi slopes pre-scaled by 1/ln 2 (the kernels work in log2 space), and a
zero output when there is no metadata (profiling runs).

MI355X specifics:
  * the KV-cache write (do_kv_cache_update) is this build's own HIP scatter,
    torch.ops.fxpr.reshape_and_cache, not vLLM's compiled extension;
  * the metadata (query_start_loc, seq_lens, block_table, max_query_len,
    slot_mapping) is the same structure vLLM's own paged backends build; it
    is borrowed from the first backend of vLLM's ROCm-capable set that
    imports (ROCm paged attention, Triton, FlashAttention).

Requires vLLM (imported at module load, as in the reference).
"""

from __future__ import annotations

import importlib
import logging
from typing import ClassVar

import torch
from vllm.config.cache import CacheDType
from vllm.v1.attention.backend import (
    AttentionBackend,
    AttentionImpl,
    AttentionLayer,
    AttentionMetadata,
    AttentionMetadataBuilder,
    AttentionType,
    MultipleOf,
)

from . import _lib  # noqa: F401  (registers torch.ops.fxpr.*)
from .config import get_runtime_config

logger = logging.getLogger("fxpr_vllm")

RCP_LN2 = 1.4426950408889634

# (module, metadata class, builder class), first importable wins
_METADATA_SOURCES = (
    ("vllm.v1.attention.backends.rocm_attn", "RocmAttentionMetadata", "RocmAttentionMetadataBuilder"),
    ("vllm.v1.attention.backends.triton_attn", "TritonAttentionMetadata", "TritonAttentionMetadataBuilder"),
    ("vllm.v1.attention.backends.flash_attn", "FlashAttentionMetadata", "FlashAttentionMetadataBuilder"),
)
_metadata_classes: tuple[type, type] | None = None


def _metadata_pair() -> tuple[type, type]:
    global _metadata_classes
    if _metadata_classes is None:
        errors = []
        for mod_name, meta, builder in _METADATA_SOURCES:
            try:
                mod = importlib.import_module(mod_name)
                _metadata_classes = (getattr(mod, meta), getattr(mod, builder))
                break
            except (ImportError, AttributeError) as e:
                errors.append(f"{mod_name}: {e}")
        else:
            raise ImportError("no vLLM paged-attention metadata builder importable: " + "; ".join(errors))
    return _metadata_classes


class DeterministicAttentionBackend(AttentionBackend):
    accept_output_buffer: bool = True
    supported_dtypes: ClassVar[list[torch.dtype]] = [torch.float16, torch.bfloat16, torch.float32]
    supported_kv_cache_dtypes: ClassVar[list[CacheDType]] = ["auto", "float16", "bfloat16"]
    forward_includes_kv_cache_update: bool = False

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_supported_kernel_block_sizes() -> list[int | MultipleOf]:
        return [MultipleOf(16)]

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "auto") -> tuple[int, ...]:
        if block_size % 16 != 0:
            raise ValueError("Block size must be a multiple of 16.")
        return (num_blocks, 2, block_size, num_kv_heads, head_size)

    @staticmethod
    def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple[int, ...]:
        return (1, 0, 2, 3, 4, 5) if include_num_layers_dimension else (0, 1, 2, 3, 4)

    @staticmethod
    def use_cascade_attention(*args, **kwargs) -> bool:
        return False

    @staticmethod
    def get_impl_cls() -> type["DeterministicAttentionImpl"]:
        return DeterministicAttentionImpl

    @staticmethod
    def get_metadata_cls() -> type[AttentionMetadata]:
        return _metadata_pair()[0]

    @staticmethod
    def get_builder_cls() -> type[AttentionMetadataBuilder]:
        return _metadata_pair()[1]

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        # 16-bit caches: head_size % 8 == 0 and <= 256 (fp32: <= 128), and the
        # reference's lower bound of 32
        return 32 <= head_size <= 256 and head_size % 8 == 0


class DeterministicAttentionImpl(AttentionImpl):
    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: list[float] | None, sliding_window: int | None,
                 kv_cache_dtype: str = "auto", logits_soft_cap: float | None = None,
                 attn_type: AttentionType | None = AttentionType.DECODER, *_extra_positional,
                 **kwargs) -> None:
        if attn_type is not None and attn_type != AttentionType.DECODER:
            raise NotImplementedError(
                f"DeterministicAttention only supports decoder attention; got attn_type={attn_type!r}.")
        if kv_cache_dtype not in ("auto", "fp16", "bf16"):
            raise NotImplementedError(
                f"DeterministicAttention does not support kv_cache_dtype={kv_cache_dtype!r}; "
                "supported: auto, fp16, bf16.")
        cfg = get_runtime_config()
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.num_kv_groups = num_heads // num_kv_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.logits_soft_cap = float(logits_soft_cap) if logits_soft_cap else 0.0
        self.window_size = int(sliding_window) if sliding_window else 0
        self.attn_type = attn_type or AttentionType.DECODER
        self.fxp_int_bits = cfg.fxp_int_bits
        self.fxp_frac_bits = cfg.fxp_frac_bits
        self.alibi_slopes: torch.Tensor | None = None
        if alibi_slopes is not None:
            slopes = torch.tensor(alibi_slopes, dtype=torch.float32) * RCP_LN2
            if slopes.shape != (num_heads,):
                raise ValueError(f"alibi_slopes shape {tuple(slopes.shape)} != (num_heads={num_heads},)")
            self.alibi_slopes = slopes

    def forward(self, layer: AttentionLayer, query: torch.Tensor, key: torch.Tensor,
                value: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: AttentionMetadata | None,
                output: torch.Tensor | None = None, output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None, **kwargs) -> torch.Tensor:
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("DeterministicAttention does not support fp8/quantized output scales.")
        from .warmup import warmup_attention

        warmup_attention(self.num_heads, self.num_kv_heads, self.head_size, kv_cache.dtype, query.device,
                         self.window_size, self.logits_soft_cap, self.fxp_int_bits, self.fxp_frac_bits)
        num_tokens = query.shape[0]
        query = query.view(num_tokens, self.num_heads, self.head_size)
        if output is None:
            output = torch.empty(num_tokens, self.num_heads, self.head_size, dtype=query.dtype,
                                 device=query.device)
        else:
            output = output.view(num_tokens, self.num_heads, self.head_size)
        if attn_metadata is None:  # profiling run
            output.zero_()
            return output.view(num_tokens, self.num_heads * self.head_size)

        if self.alibi_slopes is not None and self.alibi_slopes.device != query.device:
            self.alibi_slopes = self.alibi_slopes.to(query.device)
        qsl = attn_metadata.query_start_loc
        if qsl.dtype != torch.int32:
            qsl = qsl.to(torch.int32)
        seq_lens = attn_metadata.seq_lens
        if seq_lens.dtype != torch.int32:
            seq_lens = seq_lens.to(torch.int32)
        q_in = query if query.dtype == kv_cache.dtype else query.to(kv_cache.dtype)
        out = output if output.dtype == q_in.dtype else torch.empty_like(q_in)
        torch.ops.fxpr.unified_attention_fxp(
            q_in, kv_cache, out, qsl, seq_lens, attn_metadata.block_table,
            int(attn_metadata.max_query_len), self.alibi_slopes, True, float(self.scale),
            int(self.fxp_int_bits), int(self.fxp_frac_bits), float(self.logits_soft_cap),
            int(self.window_size), 0)
        if out is not output:
            output.copy_(out)
        return output.view(num_tokens, self.num_heads * self.head_size)

    def do_kv_cache_update(self, layer: AttentionLayer, key: torch.Tensor, value: torch.Tensor,
                           kv_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        if self.attn_type in (AttentionType.ENCODER_ONLY, AttentionType.ENCODER):
            return
        num_tokens = key.shape[0]
        torch.ops.fxpr.reshape_and_cache(
            key.view(num_tokens, self.num_kv_heads, self.head_size),
            value.view(num_tokens, self.num_kv_heads, self.head_size),
            kv_cache, slot_mapping)
