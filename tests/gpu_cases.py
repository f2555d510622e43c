"""Shared builders for the GPU parity tests (imported by tests/test_gpu_*.py).

Caches are built on the GPU with the store kernel (bit-exact to the oracle,
tests/test_gpu_store.py) and copied back as the oracle's byte blob, so the
oracle and the kernel attend over the same quantized cache.
"""
from __future__ import annotations

import numpy as np
import torch

from k8v4_v030.cache_views import bind_regions
from k8v4_v030.layout import PAGE, PageLayout
from oracle import paged

DEV = "cuda"

# Attention tolerance: max-abs 2e-3 with a 1e-2 relative allowance.
ATOL, RTOL = 2e-3, 1e-2


def assert_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), "%s: non-finite output" % what
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), "%s: max abs err %.3g at %s (want %.4g got %.4g)" % (
        what, err.max(), np.unravel_index(err.argmax(), err.shape),
        want.flat[err.argmax()], got.flat[err.argmax()])
    return float(err.max())


def max_abs(a, b) -> float:
    return float((torch.as_tensor(a).double() - torch.as_tensor(b).double()).abs().max())


class Cache:
    """A zeroed paged cache on the GPU plus its region views."""

    def __init__(self, num_pages: int, layout: PageLayout):
        self.layout = layout
        self.num_pages = num_pages
        self.raw = torch.zeros(num_pages * layout.page_bytes, dtype=torch.int8, device=DEV)
        self.views = bind_regions(self.raw, layout)
        self.geom = paged.Geometry(layout.hkv, layout.head_dim)

    def store(self, ops, k, v, slots):
        v_ = self.views
        ops.kv_store_paged(k, v, slots, v_["k"], v_["k_scale"], v_["v"], v_["v_scale"], v_["v_zero"])

    def blob(self) -> np.ndarray:
        torch.cuda.synchronize()
        return self.raw.view(torch.uint8).cpu().numpy()

    def region_args(self):
        v_ = self.views
        return v_["k"], v_["k_scale"], v_["v"], v_["v_scale"], v_["v_zero"]


def seeded_normal(gen: torch.Generator, shape, chunk=4096) -> torch.Tensor:
    """fp16 N(0,1) filled in token chunks (keeps host memory flat for long sequences)."""
    out = torch.empty(shape, dtype=torch.float16)
    for s in range(0, shape[0], chunk):
        e = min(shape[0], s + chunk)
        out[s:e] = torch.randn((e - s,) + tuple(shape[1:]), generator=gen, dtype=torch.float16)
    return out


def fill_sequence(ops, cache: Cache, gen, table_row, length: int, ppb: int = 1, start: int = 0):
    """Store ``length`` N(0,1) tokens for one sequence through its block-table row."""
    lay = cache.layout
    row = torch.as_tensor(table_row, dtype=torch.int64)
    for s in range(start, length, 65536):
        e = min(length, s + 65536)
        t = torch.arange(s, e)
        p = t // PAGE
        phys = row[p // ppb] * ppb + p % ppb
        slots = (phys * PAGE + t % PAGE).to(DEV)
        k = seeded_normal(gen, (e - s, lay.hkv, lay.head_dim)).to(DEV)
        v = seeded_normal(gen, (e - s, lay.hkv, lay.head_dim)).to(DEV)
        cache.store(ops, k, v, slots)


def decode(ops, cache: Cache, q, block_table, seq_lens, q_len, ppb=1, visible=None,
           out_dtype=torch.float16, num_splits=0):
    """Run the batch decode op with a right-sized workspace; returns the output tensor."""
    lay = cache.layout
    bt = block_table.to(device=DEV, dtype=torch.int32)
    sl = seq_lens.to(device=DEV, dtype=torch.int32)
    batch = bt.shape[0]
    nbytes = ops.attn_workspace_bytes(batch, bt.shape[1], ppb, q_len, lay.hkv, lay.head_dim, num_splits)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=DEV)
    out = torch.full(q.shape, float("nan"), dtype=out_dtype, device=DEV)
    vis = None if visible is None else visible.to(device=DEV, dtype=torch.int32)
    ops.int8k_int4v_attn_batch(q.to(DEV), None, None, *cache.region_args(), bt, sl, vis, ws,
                               None, None, None, out, q_len, ppb, num_splits=num_splits)
    torch.cuda.synchronize()
    return out


def random_tables(gen, lengths, pool_pages, ppb=1, width=None):
    """Distinct random table entries (manager blocks of ``ppb`` pages) for each sequence."""
    blocks = [-(-((L + PAGE - 1) // PAGE) // ppb) for L in lengths]
    width = width or max(max(blocks), 1)
    pool_blocks = pool_pages // ppb
    perm = torch.randperm(pool_blocks, generator=gen)
    assert sum(blocks) <= pool_blocks
    table = torch.zeros((len(lengths), width), dtype=torch.int32)
    cur = 0
    for b, n in enumerate(blocks):
        table[b, :n] = perm[cur : cur + n].to(torch.int32)
        cur += n
    return table
