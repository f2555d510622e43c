"""The reference's eager prefill entry point, served by the HIP prefill kernel.

Reference: k8v4_v030/dequant.py:213-242 (``eager_prefill``: gather and
dequantize the pages, then bottom-right causal SDPA, key-tiled for long
sequences).  Callers that import it from this module name get the same
arguments, return value and errors; the gather, dequantization and attention
all run in ``k8v4_prefill_paged`` (one launch sequence over every KV head).
"""
from __future__ import annotations

import torch

from .prefill import hip_prefill


def eager_prefill(
    query: torch.Tensor,
    views: dict[str, torch.Tensor],
    block_row: torch.Tensor,
    seq_len: int,
    pages_per_block: int,
    scale: float,
) -> torch.Tensor:
    """Bottom-right causal attention of the last ``q_len`` tokens of a sequence:
    ``[q_len, 6 * hkv, D]`` in the query's dtype; an empty query returns
    itself; a query longer than the sequence or with another head count than
    the cache's raises ``RuntimeError`` (dequant.py:223-234)."""
    return hip_prefill(query, views, block_row, seq_len, pages_per_block, scale)


__all__ = ["eager_prefill"]
