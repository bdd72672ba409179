from dataclasses import dataclass

import torch

from ..backend import AttentionMetadata, AttentionMetadataBuilder


@dataclass
class TritonAttentionMetadata(AttentionMetadata):
    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor


class TritonAttentionMetadataBuilder(AttentionMetadataBuilder):
    pass
