"""Chunked prefill over the quantized paged cache on the HIP kernel.

``hip_prefill`` takes the arguments of the reference's prefill entry points
(``eager_prefill``, k8v4_v030/dequant.py:213-242, and ``head_major_prefill``,
onednn_prefill.py:188-241) and returns the same ``[q_len, HQ, D]`` tensor in
the query's dtype, with the same errors: an empty query returns itself, a
query longer than the sequence or with a head count the cache does not hold
raises ``RuntimeError``.
"""
from __future__ import annotations

import torch

from .layout import GQA
from .ops_api import ops


def views_hkv(views: dict[str, torch.Tensor]) -> int:
    """KV heads of a ``bind_regions`` view dict (its k view is ``[P, 64, hkv, D]``)."""
    return int(views["k"].shape[2])


def hip_prefill(
    query: torch.Tensor,
    views: dict[str, torch.Tensor],
    block_row: torch.Tensor,
    seq_len: int,
    pages_per_block: int,
    scale: float,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Bottom-right causal attention of the last ``q_len`` tokens of a sequence."""
    q_len = int(query.shape[0])
    seq_len = int(seq_len)
    if q_len == 0:
        return query
    if q_len > seq_len:
        raise RuntimeError("query longer than the KV sequence")
    hkv = views_hkv(views)
    if int(query.shape[1]) != GQA * hkv:
        raise RuntimeError(
            "query has %d heads, the K8/V4 cache holds %d (needs %d)" % (int(query.shape[1]), hkv, GQA * hkv)
        )
    if out is None:
        out = torch.empty_like(query)
    row = block_row
    if row.dtype != torch.int32 or not row.is_contiguous():
        row = row.to(torch.int32).contiguous()
    ops().prefill_paged(query, views["k"], views["k_scale"], views["v"], views["v_scale"], views["v_zero"],
                        row, seq_len, pages_per_block, scale, out, workspace)
    return out


__all__ = ["hip_prefill", "views_hkv"]
