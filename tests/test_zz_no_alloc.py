"""The allocation-free decode entry point against the workspace one (GPU).

``k8v4_attn_batch_noalloc`` keeps its split states in a library-owned device
buffer; ``k8v4_attn_batch`` takes a caller workspace.  Both run the same
kernels with the same grid, so two calls in a row -- the second with a smaller
input, over the buffer the first one left behind -- give the same bytes as
the workspace entry point.  A call needing more split states than the buffer
holds is refused before anything is launched.
"""
from __future__ import annotations

import pytest
import torch

from gpu_cases import DEV, Cache, fill_sequence, random_tables, seeded_normal
from k8v4_v030 import ops_api
from k8v4_v030.layout import PageLayout

pytestmark = pytest.mark.gpu


def _args(cache, q, table, seq, q_len, out):
    """k8v4_attn_batch arguments up to out_tok_stride (the shared prefix of both entry points)."""
    lay = cache.layout
    return [ops_api._ptr(q), ops_api.F16, int(q.stride(0)),
            *ops_api.cache_args(*cache.region_args()),
            ops_api._ptr(table), int(table.stride(0)), int(table.shape[1]), 1, ops_api._ptr(seq), None, 0,
            int(table.shape[0]), q_len, lay.hkv, lay.head_dim, ops_api._ptr(out), ops_api.F32, int(out.stride(0))]


def _both(lib, cache, q, table, seq, q_len):
    stream = torch.cuda.current_stream().cuda_stream
    with_ws = torch.full(q.shape, float("nan"), dtype=torch.float32, device=DEV)
    nbytes = lib.k8v4_attn_workspace_bytes(int(table.shape[0]), int(table.shape[1]), 1, q_len, cache.layout.hkv,
                                           cache.layout.head_dim, 0)
    ws = torch.empty(nbytes // 4 + 4, dtype=torch.float32, device=DEV)
    rc = lib.k8v4_attn_batch(*_args(cache, q, table, seq, q_len, with_ws), ops_api._ptr(ws), ws.numel() * 4, 0, stream)
    assert rc == 0, lib.k8v4_last_error()
    no_ws = torch.full(q.shape, float("nan"), dtype=torch.float32, device=DEV)
    rc = lib.k8v4_attn_batch_noalloc(*_args(cache, q, table, seq, q_len, no_ws), 0, stream)
    assert rc == 0, lib.k8v4_last_error()
    torch.cuda.synchronize()
    return with_ws, no_ws


@pytest.mark.parametrize("hkv,d", [(4, 128), (2, 256), (4, 256)])
def test_noalloc_entry_matches_the_workspace_entry_on_two_calls(hkv, d):
    """(4, 128): split states only; (2, 256) and (4, 256): the paired-halves
    layout, whose query tile sits ahead of the split states in the same
    buffer."""
    lib = ops_api.load_library()
    print("noalloc hkv=%d d=%d: first call (2 x 20,000, q=7)" % (hkv, d), flush=True)
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(777 + d)
    lengths = [20000, 17000]
    table = random_tables(gen, lengths, 700)
    cache = Cache(700, lay)
    for b, L in enumerate(lengths):
        fill_sequence(ops_api.ops(), cache, gen, table[b], L)
    q = seeded_normal(gen, (2 * 7, lay.hq, d)).to(DEV)
    tbl = table.to(DEV)
    seq = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    a, b = _both(lib, cache, q, tbl, seq, 7)
    assert torch.isfinite(a).all() and torch.equal(a, b)
    print("noalloc hkv=%d d=%d: second call (1 x 3,000, q=3)" % (hkv, d), flush=True)
    q2 = seeded_normal(gen, (1 * 3, lay.hq, d)).to(DEV)
    seq2 = torch.tensor([3000], dtype=torch.int32, device=DEV)
    a2, b2 = _both(lib, cache, q2, tbl[:1].contiguous(), seq2, 3)
    assert torch.isfinite(a2).all() and torch.equal(a2, b2)


def test_noalloc_entry_refuses_calls_beyond_its_buffer():
    lib = ops_api.load_library()
    cap = lib.k8v4_attn_noalloc_max_bytes()
    assert cap == 32 << 20
    lay = PageLayout(2, 256)
    cache = Cache(4, lay)
    q = torch.zeros((2000 * 10, 12, 256), dtype=torch.float16, device=DEV)
    out = torch.zeros(q.shape, dtype=torch.float32, device=DEV)
    table = torch.zeros((2000, 4), dtype=torch.int32, device=DEV)
    seq = torch.ones(2000, dtype=torch.int32, device=DEV)
    assert lib.k8v4_attn_workspace_bytes(2000, 4, 1, 10, 2, 256, 0) > cap
    rc = lib.k8v4_attn_batch_noalloc(*_args(cache, q, table, seq, 10, out), 0,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 2 and b"holds %d" % cap in lib.k8v4_last_error()
