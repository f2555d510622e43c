"""Zero-copy region views over one layer's KV allocation.

vLLM hands each layer a byte tensor shaped ``[block, head, token, cell]`` whose
memory order is ``[block, token, head, cell]``.  Kernel pages are that span in
*address* order, so the views here are built from the raw bytes, never from a
logical ``.contiguous()`` (which would permute bytes and split pages).

Reference: k8v4_v030/cache_views.py:28-109 (``memory_order_bytes``,
``bind_regions``), same refusal rules: non-byte dtype, empty, gapped,
overlapping or non-positive strides, storage offset not 4-byte aligned, a
length that is not a whole number of pages, and a head count that disagrees
with the layout.
"""
from __future__ import annotations

import torch

from .layout import PageLayout, region_view_specs

_BYTE_DTYPES = (torch.int8, torch.uint8)


def _not_dense(kv_cache: torch.Tensor) -> RuntimeError:
    return RuntimeError(
        "K8/V4 layer cache is not a dense byte span (shape=%s stride=%s)"
        % (tuple(kv_cache.shape), tuple(kv_cache.stride()))
    )


def memory_order_bytes(kv_cache: torch.Tensor) -> torch.Tensor:
    """The bytes of ``kv_cache`` as one int8 vector in address order (a view, no copy)."""
    if kv_cache.dtype not in _BYTE_DTYPES:
        raise RuntimeError("K8/V4 cache dtype %s is not a byte tensor" % kv_cache.dtype)
    total = int(kv_cache.numel())
    if total == 0:
        raise RuntimeError("K8/V4 cache tensor is empty")
    dims = [(int(n), int(s)) for n, s in zip(kv_cache.shape, kv_cache.stride()) if int(n) != 1]
    if any(s <= 0 for _, s in dims):
        raise _not_dense(kv_cache)
    # Sorted by stride, each dim must start exactly where the finer ones end.
    span = 1
    for n, s in sorted(dims, key=lambda item: item[1]):
        if s != span:
            raise _not_dense(kv_cache)
        span *= n
    if span != total:
        raise _not_dense(kv_cache)
    offset = int(kv_cache.storage_offset())
    if offset % 4:
        raise RuntimeError("K8/V4 cache storage is not 4-byte aligned")
    flat = torch.as_strided(kv_cache, size=(total,), stride=(1,), storage_offset=offset)
    return flat if flat.dtype == torch.int8 else flat.view(torch.int8)


def bind_regions(kv_cache: torch.Tensor, layout: PageLayout) -> dict[str, torch.Tensor]:
    """Five strided views (k, v, k_scale, v_scale, v_zero) sharing ``kv_cache`` storage."""
    if kv_cache.dim() == 4 and kv_cache.shape[1] > 1 and kv_cache.shape[1] != layout.hkv:
        raise RuntimeError(
            "K8/V4 cache has %d KV heads, layout serves %d" % (int(kv_cache.shape[1]), layout.hkv)
        )
    raw = memory_order_bytes(kv_cache)
    nbytes = int(raw.numel())
    if nbytes % layout.page_bytes:
        raise RuntimeError(
            "K8/V4 cache has %d bytes, not a multiple of the %d-byte page"
            % (nbytes, layout.page_bytes)
        )
    specs = region_view_specs(nbytes // layout.page_bytes, layout)
    base = int(raw.storage_offset())
    as_dtype = {
        "int8": (raw, 1),
        "uint8": (raw.view(torch.uint8), 1),
        "float32": (raw.view(torch.float32), 4),
    }
    views: dict[str, torch.Tensor] = {}
    for name, spec in specs.items():
        storage, elem = as_dtype[str(spec["dtype"])]
        views[name] = torch.as_strided(
            storage,
            size=spec["shape"],
            stride=spec["stride"],
            storage_offset=(base + int(spec["byte_offset"])) // elem,
        )
    return views
