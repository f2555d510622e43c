"""The reference's head-major prefill entry point, served by the HIP prefill
kernel.

Reference: k8v4_v030/onednn_prefill.py:188-241 (``head_major_prefill``: per KV
head, gather and dequantize, pad the queries to a multiple of ``bucket`` rows,
run the fused SDPA).  Same arguments, return value and errors; the HIP kernel
takes the query rows as they are, so ``bucket`` only keeps the signature.
"""
from __future__ import annotations

import torch

from .layout import PageLayout
from .prefill import hip_prefill

Q_BUCKET = 256


def head_major_prefill(
    query: torch.Tensor,
    views: dict[str, torch.Tensor],
    block_row: torch.Tensor,
    seq_len: int,
    pages_per_block: int,
    scale: float,
    bucket: int = Q_BUCKET,
) -> torch.Tensor:
    """As ``eager_prefill``; the head count is checked first, with the
    reference's message (onednn_prefill.py:199-204)."""
    del bucket
    hq = PageLayout(int(views["k"].shape[2]), int(views["k"].shape[3])).hq
    if int(query.shape[1]) != hq:
        raise RuntimeError("query has %d heads, the K8/V4 cache holds %d" % (int(query.shape[1]), hq))
    return hip_prefill(query, views, block_row, seq_len, pages_per_block, scale)


__all__ = ["Q_BUCKET", "head_major_prefill"]
