"""Attention backend base classes (vllm/v1/attention/backend.py, the members
the K8/V4 backend uses)."""
from __future__ import annotations

import dataclasses
import enum
from typing import Generic, TypeVar

import torch


class AttentionType:
    DECODER = "decoder"
    ENCODER = "encoder"
    ENCODER_ONLY = "encoder_only"
    ENCODER_DECODER = "encoder_decoder"


class AttentionCGSupport(enum.Enum):
    NEVER = 0
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    UNIFORM_BATCH = 2
    ALWAYS = 3


@dataclasses.dataclass(frozen=True)
class MultipleOf:
    base: int


class AttentionMetadata:
    pass


M = TypeVar("M")


class AttentionMetadataBuilder(Generic[M]):
    _cudagraph_support = AttentionCGSupport.NEVER

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names
        self.vllm_config = vllm_config
        self.device = device
        self.kernel_block_size = None
        self.reorder_batch_threshold = None
        self.supports_spec_as_decode = False

    def _init_reorder_batch_threshold(self, reorder_batch_threshold=1, supports_spec_as_decode=False):
        self.reorder_batch_threshold = reorder_batch_threshold
        self.supports_spec_as_decode = supports_spec_as_decode

    def set_kernel_block_size(self, kernel_block_size):
        self.kernel_block_size = kernel_block_size


class AttentionImpl(Generic[M]):
    pass


class AttentionBackend:
    accept_output_buffer: bool = False


@dataclasses.dataclass
class CommonAttentionMetadata:
    query_start_loc: torch.Tensor
    query_start_loc_cpu: torch.Tensor
    seq_lens: torch.Tensor
    seq_lens_cpu_upper_bound: torch.Tensor | None
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    block_table_tensor: torch.Tensor
    slot_mapping: torch.Tensor
