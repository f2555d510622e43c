"""The reference's prefill entry points under their reference module names
(CPU: argument checks, which run before any library call).

Reference: k8v4_v030/dequant.py:213-234 (``eager_prefill``) and
k8v4_v030/onednn_prefill.py:188-210 (``head_major_prefill``): an empty query
comes back as is, a query longer than the sequence or with another head count
than the cache's raises ``RuntimeError`` with the reference's messages.
"""
from __future__ import annotations

import pytest
import torch

from k8v4_v030.cache_views import bind_regions
from k8v4_v030.dequant import eager_prefill
from k8v4_v030.layout import PageLayout
from k8v4_v030.onednn_prefill import Q_BUCKET, head_major_prefill


def _views(hkv=4, d=128, pages=4):
    lay = PageLayout(hkv, d)
    return bind_regions(torch.zeros(pages * lay.page_bytes, dtype=torch.int8), lay)


@pytest.mark.parametrize("entry", [eager_prefill, head_major_prefill])
def test_empty_query_returns_itself(entry):
    q = torch.zeros(0, 24, 128, dtype=torch.float16)
    assert entry(q, _views(), torch.arange(4, dtype=torch.int32), 10, 1, 0.1) is q


@pytest.mark.parametrize("entry", [eager_prefill, head_major_prefill])
def test_query_longer_than_the_sequence(entry):
    q = torch.zeros(10, 24, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="query longer than the KV sequence"):
        entry(q, _views(), torch.arange(4, dtype=torch.int32), 9, 1, 0.1)


def test_head_count_messages():
    q = torch.zeros(10, 12, 128, dtype=torch.float16)
    row = torch.arange(4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match=r"query has 12 heads, the K8/V4 cache holds 4 \(needs 24\)"):
        eager_prefill(q, _views(), row, 100, 1, 0.1)
    with pytest.raises(RuntimeError, match=r"query has 12 heads, the K8/V4 cache holds 24$"):
        head_major_prefill(q, _views(), row, 100, 1, 0.1)
    # head_major_prefill checks the heads before the lengths (onednn_prefill.py:199-210).
    with pytest.raises(RuntimeError, match="holds 24"):
        head_major_prefill(torch.zeros(0, 12, 128, dtype=torch.float16), _views(), row, 100, 1, 0.1)
    assert Q_BUCKET == 256
