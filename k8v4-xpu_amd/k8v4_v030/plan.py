"""Host-side batch decisions for the packed decode path.

All inputs are host integers (the CPU copy of ``query_start_loc``), so a
captured graph never reads them back from the device.

Reference: k8v4_v030/plan.py:22-146.  Differences: the head dim is a parameter
(128 or 256) instead of the fixed 256, and ``attn_workspace_bytes`` sizes the
split-K scratch of the HIP decode kernel.
"""
from __future__ import annotations

from collections.abc import Sequence

from .layout import (
    DECODE_MAX_T,
    D,
    GQA,
    PAGE,
    SUPPORTED_HEAD_DIMS,
    PageLayout,
    attention_pages_per_block,
    max_kernel_pages,
)


def query_lengths(starts: Sequence[int]) -> list[int]:
    """Per-request query lengths from an inclusive ``query_start_loc``."""
    if len(starts) < 2:
        raise ValueError("query_start_loc needs a start and an end")
    out = []
    for lo, hi in zip(starts[:-1], starts[1:]):
        n = int(hi) - int(lo)
        if n < 0:
            raise ValueError("query_start_loc decreased")
        out.append(n)
    return out


def uniform_packed_q_len(starts: Sequence[int]) -> int:
    """The common query length if every request has it and it fits the decode tile, else 0."""
    lengths = query_lengths(starts)
    if not lengths:
        return 0
    q = lengths[0]
    if not 1 <= q <= DECODE_MAX_T or any(n != q for n in lengths):
        return 0
    return q


def query_segments(starts: Sequence[int]) -> list[tuple[int, int, int]]:
    """Maximal runs of equal query length as ``(first_request, count, q_len)``."""
    lengths = query_lengths(starts)
    runs: list[tuple[int, int, int]] = []
    for i, n in enumerate(lengths):
        if runs and runs[-1][2] == n:
            first, count, _ = runs[-1]
            runs[-1] = (first, count + 1, n)
        else:
            runs.append((i, 1, n))
    return runs


def token_span(starts: Sequence[int], first_request: int, count: int, q_len: int) -> tuple[int, int]:
    """(token offset, token count) of a tightly packed run of requests."""
    if count < 1 or q_len < 1:
        raise ValueError("empty segment")
    if first_request < 0 or first_request + count >= len(starts):
        raise ValueError("segment outside query_start_loc")
    t0 = int(starts[first_request])
    t1 = int(starts[first_request + count])
    if t1 - t0 != count * q_len:
        raise ValueError("query segment is not tightly packed")
    return t0, t1 - t0


def scratch_capacity(
    max_model_len: int,
    manager_block: int,
    kernel_block: int | None,
    max_batched_tokens: int,
    max_seqs: int,
    capture_sizes: Sequence[int],
    layout: PageLayout,
) -> tuple[int, int, int]:
    """``(nprog_max, max_store_tokens, max_out_tokens)`` for one worker.

    One extra table entry's pages is margin past a full context; the output
    buffer covers the widest capture size and a full decode batch.
    """
    ratio = attention_pages_per_block(manager_block, kernel_block)
    pages = max_kernel_pages(max_model_len, manager_block, kernel_block) + ratio
    widest = max([int(s) for s in capture_sizes] + [0])
    max_out = max(int(max_seqs) * DECODE_MAX_T, widest, DECODE_MAX_T)
    if int(max_batched_tokens) < 1:
        raise ValueError("max_batched_tokens")
    return pages * layout.hkv, int(max_batched_tokens), max_out


def workspace_programs(table_width: int, pages_per_block: int, layout: PageLayout) -> int:
    """Split programs the reference sized its per-request workspace for (pages * hkv)."""
    w, r = int(table_width), int(pages_per_block)
    if w < 1 or r < 1:
        raise ValueError("workspace shape")
    return w * r * layout.hkv


def split_state_bytes(q_len: int, layout: PageLayout) -> int:
    """Bytes of one split's state: per KV head and live row, D fp16 outputs, then fp32 m and l."""
    rows = int(q_len) * GQA
    return layout.hkv * rows * (2 * layout.head_dim + 8)


def query_tile_bytes(batch: int, layout: PageLayout) -> int:
    """Workspace head of a 256-dim decode (two or four KV heads: its query runs
    through a quantization kernel first): per sequence and KV head 64 rows of
    int8 codes, then their fp32 scales, each part rounded up to 256 bytes; 0
    otherwise."""
    if not (layout.head_dim == 256 and layout.hkv in (2, 4)):
        return 0
    rows = int(batch) * layout.hkv * PAGE
    return -(-rows * layout.head_dim // 256) * 256 + -(-rows * 4 // 256) * 256


def attn_workspace_bytes(max_splits: int, q_len: int, layout: PageLayout, batch: int = 1) -> int:
    """Scratch the decode kernel needs for ``max_splits`` split-K work-groups over ``batch`` sequences."""
    return query_tile_bytes(batch, layout) + int(max_splits) * split_state_bytes(q_len, layout)


def layout_for_heads(num_heads: int, num_kv_heads: int, head_size: int) -> PageLayout:
    """Validated layout for one rank, or a RuntimeError naming what is wrong."""
    if int(head_size) not in SUPPORTED_HEAD_DIMS:
        raise RuntimeError(
            "K8/V4 kernel head dim is one of %s, got %s" % (SUPPORTED_HEAD_DIMS, head_size)
        )
    try:
        return PageLayout.for_heads(num_heads, num_kv_heads, int(head_size))
    except ValueError as error:
        raise RuntimeError(str(error)) from error


def require_decoder(
    attn_type: object,
    sliding_window: int | None,
    alibi_slopes: object,
    logits_soft_cap: float | None,
    scale: float,
    head_dim: int = D,
) -> None:
    """Refuse attention variants the kernels do not implement; the scale is fixed at 1/sqrt(D)."""
    kind = getattr(attn_type, "value", attn_type)
    if str(kind) != "decoder":
        raise RuntimeError("K8/V4 attention is decoder-only, got %s" % attn_type)
    if sliding_window is not None and int(sliding_window) > 0:
        raise RuntimeError("K8/V4 does not implement sliding window")
    if alibi_slopes is not None:
        raise RuntimeError("K8/V4 does not implement alibi")
    if logits_soft_cap not in (None, 0, 0.0):
        raise RuntimeError("K8/V4 does not implement logits soft cap")
    want = 1.0 / float(head_dim) ** 0.5
    if abs(float(scale) - want) > 1e-5:
        raise RuntimeError("K8/V4 kernel scale is fixed at %s, got %s" % (want, scale))


__all__ = [
    "PAGE",
    "attn_workspace_bytes",
    "query_tile_bytes",
    "layout_for_heads",
    "query_lengths",
    "query_segments",
    "require_decoder",
    "scratch_capacity",
    "split_state_bytes",
    "token_span",
    "uniform_packed_q_len",
    "workspace_programs",
]
