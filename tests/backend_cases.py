"""Shared setup for the vLLM backend tests (imported by tests/test_backend.py
and tests/test_gpu_backend.py).

vLLM is not installed in this image: when ``import vllm`` fails, the stand-in
under ``tests/vllm_stub`` (the members of vLLM 0.30's attention interface the
backend imports) is put on ``sys.path`` first.
"""
from __future__ import annotations

import math
import sys
from pathlib import Path
from types import SimpleNamespace

import torch

try:  # a real vLLM takes precedence
    import vllm  # noqa: F401
except ImportError:
    sys.path.insert(0, str(Path(__file__).resolve().parent / "vllm_stub"))

from vllm.v1.attention.backend import AttentionType, CommonAttentionMetadata  # noqa: E402
from vllm.v1.kv_cache_interface import AttentionSpec  # noqa: E402

from k8v4_v030 import backend  # noqa: E402
from k8v4_v030.layout import CACHE_DTYPE, PAGE, PageLayout  # noqa: E402


def vllm_config(max_model_len=4096, max_batched=2048, max_seqs=8, capture=(1, 2, 4, 8)):
    return SimpleNamespace(
        model_config=SimpleNamespace(max_model_len=max_model_len),
        scheduler_config=SimpleNamespace(max_num_batched_tokens=max_batched, max_num_seqs=max_seqs),
        compilation_config=SimpleNamespace(cudagraph_capture_sizes=list(capture)),
    )


def make_impl(hkv=4, head=128, **kw):
    args = dict(num_heads=6 * hkv, head_size=head, scale=1.0 / math.sqrt(head), num_kv_heads=hkv,
                kv_cache_dtype=CACHE_DTYPE)
    args.update(kw)
    return backend.Xe2K8V4Impl(**args)


def make_builder(hkv=4, head=128, block_size=64, kernel_block=64, device="cpu", **cfg):
    spec = AttentionSpec(block_size=block_size, num_kv_heads=hkv, head_size=head)
    b = backend.Xe2K8V4MetadataBuilder(spec, ["layer.0"], vllm_config(**cfg), torch.device(device))
    if kernel_block is not None:
        b.set_kernel_block_size(kernel_block)
    return b


def common_metadata(q_lens, seq_lens, block_table, slot_mapping, device):
    """vLLM's per-step metadata for requests with the given query and total lengths."""
    starts = [0]
    for q in q_lens:
        starts.append(starts[-1] + int(q))
    loc = torch.tensor(starts, dtype=torch.int32)
    lens = torch.tensor(seq_lens, dtype=torch.int32)
    return CommonAttentionMetadata(
        query_start_loc=loc.to(device),
        query_start_loc_cpu=loc,
        seq_lens=lens.to(device),
        seq_lens_cpu_upper_bound=lens,
        num_reqs=len(q_lens),
        num_actual_tokens=starts[-1],
        max_query_len=max(q_lens),
        max_seq_len=max(seq_lens),
        block_table_tensor=block_table.to(device=device, dtype=torch.int32),
        slot_mapping=slot_mapping.to(device=device, dtype=torch.int64),
    )


def vllm_cache(num_blocks, block_tokens, layout: PageLayout, device):
    """A live layer the way vLLM allocates it: ``[block, kv_head, token, slot_bytes]`` int8.

    Its bytes in memory order are the reference's region-major pages."""
    return torch.zeros((num_blocks, layout.hkv, block_tokens, layout.slot_bytes_per_head), dtype=torch.int8,
                       device=device)


def slots_for(table_row, positions, block_tokens):
    row = torch.as_tensor(table_row, dtype=torch.int64)
    pos = torch.as_tensor(positions, dtype=torch.int64)
    return row[pos // block_tokens] * block_tokens + pos % block_tokens


__all__ = ["AttentionType", "PAGE", "backend", "common_metadata", "make_builder", "make_impl", "slots_for",
           "vllm_cache", "vllm_config"]
