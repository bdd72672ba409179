"""The CUSTOM attention backend: vLLM attention on torch.ops.fxpr.unified_attention_fxp.

vLLM talks to a backend through the AttentionBackend / AttentionImpl
interface; the class names, the interface members and what each accepts or
rejects follow the reference backend (fxpr_vllm/attention_backend.py:40-277
of Gursukh/vLLM-Triton-Fixed-Point-Reductions), so selecting
attention_backend="CUSTOM" gives the same behaviour:

  * decoder self-attention only; fp16 / bf16 / fp32 activations; KV cache
    "auto" / fp16 / bf16 (no fp8, no quantised output scales);
  * KV cache [num_blocks, 2, page, num_kv_heads, head_size], pages a
    multiple of 16 keys; causal, with the op's automatic KV-split count;
  * ALiBi slopes given per natural-log unit are converted to the kernels'
    log2 units; a call without metadata (vLLM's profiling run) returns
    zeros.

How this backend differs from the reference's:
  * the KV-cache write (do_kv_cache_update) is this library's HIP scatter,
    torch.ops.fxpr.reshape_and_cache, rather than vLLM's compiled
    reshape_and_cache_flash;
  * the per-step metadata (query_start_loc, seq_lens, block_table,
    max_query_len, slot_mapping) has the layout vLLM's own paged backends
    build; metadata_classes() takes the classes from the first of vLLM's
    ROCm-capable backends that imports;
  * a caller's output buffer is always the one written (a dtype mismatch goes
    through a temporary and a copy into it).

Importing this module requires vLLM.
"""

from __future__ import annotations

import functools
import importlib
import logging
from dataclasses import dataclass
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

# scores are formed in log2 units (exp2 of the scaled logits), so a bias
# given per natural-log unit is multiplied by log2(e)
LOG2E = 1.4426950408889634

PAGE_MULTIPLE = 16
ACCEPTED_KV_CACHE_DTYPES = ("auto", "fp16", "bf16")   # vLLM's kv_cache_dtype strings

# (module, metadata class, builder class), in order of preference on ROCm
METADATA_PROVIDERS = (
    ("vllm.v1.attention.backends.rocm_attn", "RocmAttentionMetadata", "RocmAttentionMetadataBuilder"),
    ("vllm.v1.attention.backends.triton_attn", "TritonAttentionMetadata", "TritonAttentionMetadataBuilder"),
    ("vllm.v1.attention.backends.flash_attn", "FlashAttentionMetadata", "FlashAttentionMetadataBuilder"),
)


@functools.lru_cache(maxsize=1)
def metadata_classes() -> tuple[type, type]:
    """(metadata class, builder class) of the first importable provider."""
    misses = []
    for module_name, meta_name, builder_name in METADATA_PROVIDERS:
        try:
            module = importlib.import_module(module_name)
        except ImportError as exc:
            misses.append(f"{module_name} ({exc})")
            continue
        meta, builder = getattr(module, meta_name, None), getattr(module, builder_name, None)
        if meta is not None and builder is not None:
            return meta, builder
        misses.append(f"{module_name} (no {meta_name} / {builder_name})")
    raise ImportError("fxpr CUSTOM backend: no vLLM paged-attention metadata provider: " + "; ".join(misses))


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
        return [MultipleOf(PAGE_MULTIPLE)]

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "auto") -> tuple[int, ...]:
        if block_size % PAGE_MULTIPLE:
            raise ValueError(f"CUSTOM attention pages hold a multiple of {PAGE_MULTIPLE} keys; "
                             f"got block_size={block_size}")
        return (num_blocks, 2, block_size, num_kv_heads, head_size)

    @staticmethod
    def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple[int, ...]:
        # the natural order; with a leading layer axis, K/V outermost
        natural = (0, 1, 2, 3, 4)
        if not include_num_layers_dimension:
            return natural
        return (1, 0) + tuple(d + 1 for d in natural[1:])

    @staticmethod
    def use_cascade_attention(*args, **kwargs) -> bool:
        return False

    @staticmethod
    def get_impl_cls() -> type["DeterministicAttentionImpl"]:
        return DeterministicAttentionImpl

    @staticmethod
    def get_metadata_cls() -> type[AttentionMetadata]:
        return metadata_classes()[0]

    @staticmethod
    def get_builder_cls() -> type[AttentionMetadataBuilder]:
        return metadata_classes()[1]

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        # the kernels take head sizes that are multiples of 8 up to 256; the
        # reference backend's lower bound is 32
        return 32 <= head_size <= 256 and head_size % 8 == 0


def _int32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


@dataclass(frozen=True)
class _Plan:
    """What every forward of one attention layer passes to the op."""

    num_heads: int
    num_kv_heads: int
    head_size: int
    scale: float
    logits_soft_cap: float      # 0 = off
    window_size: int            # 0 = unbounded
    fxp_int_bits: int
    fxp_frac_bits: int


class DeterministicAttentionImpl(AttentionImpl):
    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: list[float] | None, sliding_window: int | None,
                 kv_cache_dtype: str = "auto", logits_soft_cap: float | None = None,
                 attn_type: AttentionType | None = AttentionType.DECODER, *_extra_positional,
                 **kwargs) -> None:
        attn_type = AttentionType.DECODER if attn_type is None else attn_type
        if attn_type != AttentionType.DECODER:
            raise NotImplementedError(f"CUSTOM (fixed-point) attention runs decoder self-attention "
                                      f"only, not attn_type={attn_type!r}")
        if kv_cache_dtype not in ACCEPTED_KV_CACHE_DTYPES:
            raise NotImplementedError(f"CUSTOM (fixed-point) attention keeps a 16-bit or auto KV "
                                      f"cache ({', '.join(ACCEPTED_KV_CACHE_DTYPES)}), not "
                                      f"kv_cache_dtype={kv_cache_dtype!r}")
        cfg = get_runtime_config()
        self.plan = _Plan(num_heads=int(num_heads), num_kv_heads=int(num_kv_heads),
                          head_size=int(head_size), scale=float(scale),
                          logits_soft_cap=float(logits_soft_cap or 0.0),
                          window_size=int(sliding_window or 0),
                          fxp_int_bits=cfg.fxp_int_bits, fxp_frac_bits=cfg.fxp_frac_bits)
        self.attn_type = attn_type
        self.kv_cache_dtype = kv_cache_dtype
        self.alibi_slopes: torch.Tensor | None = None
        if alibi_slopes is not None:
            slopes = torch.as_tensor(alibi_slopes, dtype=torch.float32).reshape(-1)
            if slopes.numel() != num_heads:
                raise ValueError(f"ALiBi needs one slope per query head ({num_heads}); got {slopes.numel()}")
            self.alibi_slopes = slopes * LOG2E

    # attribute names vLLM and the reference expose on an impl
    num_heads = property(lambda self: self.plan.num_heads)
    num_kv_heads = property(lambda self: self.plan.num_kv_heads)
    head_size = property(lambda self: self.plan.head_size)
    scale = property(lambda self: self.plan.scale)
    logits_soft_cap = property(lambda self: self.plan.logits_soft_cap)
    window_size = property(lambda self: self.plan.window_size)
    fxp_int_bits = property(lambda self: self.plan.fxp_int_bits)
    fxp_frac_bits = property(lambda self: self.plan.fxp_frac_bits)
    num_kv_groups = property(lambda self: self.plan.num_heads // self.plan.num_kv_heads)

    def _slopes_on(self, device: torch.device) -> torch.Tensor | None:
        if self.alibi_slopes is not None and self.alibi_slopes.device != device:
            self.alibi_slopes = self.alibi_slopes.to(device)
        return self.alibi_slopes

    def forward(self, layer: AttentionLayer, query: torch.Tensor, key: torch.Tensor,
                value: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: AttentionMetadata | None,
                output: torch.Tensor | None = None, output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None, **kwargs) -> torch.Tensor:
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("CUSTOM (fixed-point) attention writes unscaled outputs; "
                                      "fp8 / block output scales are not supported")
        p = self.plan
        tokens = query.shape[0]
        heads3d = (tokens, p.num_heads, p.head_size)
        out3d = (torch.empty(heads3d, dtype=query.dtype, device=query.device) if output is None
                 else output.view(heads3d))
        flat = out3d.view(tokens, p.num_heads * p.head_size)
        if attn_metadata is None:                # vLLM's memory-profiling pass
            return flat.zero_()

        from .warmup import warmup_attention

        warmup_attention(p.num_heads, p.num_kv_heads, p.head_size, kv_cache.dtype, query.device,
                         p.window_size, p.logits_soft_cap, p.fxp_int_bits, p.fxp_frac_bits)
        # q, the cache and the output share one dtype in the kernels
        q = query.view(heads3d).to(kv_cache.dtype)
        dst = out3d if out3d.dtype == q.dtype else torch.empty_like(q)
        torch.ops.fxpr.unified_attention_fxp(
            q, kv_cache, dst, _int32(attn_metadata.query_start_loc), _int32(attn_metadata.seq_lens),
            attn_metadata.block_table, int(attn_metadata.max_query_len), self._slopes_on(query.device),
            True, p.scale, p.fxp_int_bits, p.fxp_frac_bits, p.logits_soft_cap, p.window_size,
            0)  # 0 splits: the op chooses
        if dst is not out3d:
            out3d.copy_(dst)
        return flat

    def do_kv_cache_update(self, layer: AttentionLayer, key: torch.Tensor, value: torch.Tensor,
                           kv_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        p = self.plan
        tokens = key.shape[0]
        torch.ops.fxpr.reshape_and_cache(key.view(tokens, p.num_kv_heads, p.head_size),
                                         value.view(tokens, p.num_kv_heads, p.head_size),
                                         kv_cache, slot_mapping)
