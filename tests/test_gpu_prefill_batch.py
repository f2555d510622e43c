"""Several sequences' prefill in one call (k8v4_prefill_paged_batch) vs the oracle (GPU).

The batched entry replaces the backend's per-request prefill loop (the
reference's backend.py:376-409, one eager_prefill per request): every
sequence's rows must equal the oracle's for that sequence alone (the float64
bottom-right causal attention of oracle/attention.py, pinned to torch SDPA in
tests/test_oracle.py), rows of the query that belong to no sequence must be
left untouched, and more sequences than one launch takes must give the same
answer as the single-sequence entry.  Tolerance: max-abs 2e-3 with a 1e-2
relative allowance.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from gpu_cases import DEV, Cache, assert_close, fill_sequence, random_tables, seeded_normal
from k8v4_v030.layout import PAGE, PageLayout
from k8v4_v030.prefill import hip_prefill
from oracle import attention

pytestmark = pytest.mark.gpu


def _setup(ops, gen, lay, q_lens, seq_lens, ppb=1, gap=3, table_order=None):
    """A shared cache with every sequence's pages (sequence i in block-table
    row table_order[i]), the packed query of all sequences (``gap`` unused
    token rows before each) and their first tokens."""
    n = len(q_lens)
    assert all(ql <= sl for ql, sl in zip(q_lens, seq_lens))
    order = list(range(n)) if table_order is None else list(table_order)
    lens_by_row = [0] * n
    for i, r in enumerate(order):
        lens_by_row[r] = seq_lens[i]
    blocks = [-(-((sl + PAGE - 1) // PAGE) // ppb) for sl in lens_by_row]
    pool = (sum(blocks) + 4) * ppb
    table = random_tables(gen, lens_by_row, pool, ppb=ppb)
    cache = Cache(pool, lay)
    for r, sl in enumerate(lens_by_row):
        if sl:
            fill_sequence(ops, cache, gen, table[r], sl, ppb=ppb)
    tok0, t = [], gap
    for ql in q_lens:
        tok0.append(t)
        t += ql + gap
    q = seeded_normal(gen, (t, lay.hq, lay.head_dim))
    return cache, table, q, tok0, order


def _batch(gpu_ops, cache, table, q, tok0, q_lens, seq_lens, rows, ppb=1, out_dtype=torch.float32):
    out = torch.full(q.shape, float("nan"), dtype=out_dtype, device=DEV)
    scale = 1.0 / math.sqrt(cache.layout.head_dim)
    gpu_ops.prefill_paged_batch(q.to(DEV), *cache.region_args(), table.to(device=DEV, dtype=torch.int32), tok0,
                                q_lens, seq_lens, rows, ppb, scale, out)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _oracle(cache, q, row, seq_len, ppb=1):
    scale = 1.0 / math.sqrt(cache.layout.head_dim)
    return attention.prefill_attention(q.float().cpu().numpy(), cache.blob(), cache.geom, row.numpy(), seq_len,
                                       ppb, scale)


@pytest.mark.parametrize("hkv,d,ppb", [(4, 128, 1), (2, 128, 2), (2, 256, 1), (4, 256, 1)])
def test_batch_matches_the_oracle_per_sequence(gpu_ops, hkv, d, ppb):
    """Mixed chunk lengths (1 to 170 tokens) over short and longer contexts,
    block-table rows in another order than the query rows."""
    print("prefill batch hkv=%d d=%d ppb=%d" % (hkv, d, ppb), flush=True)
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(101 * hkv + d + ppb)
    q_lens = [1, 7, 40, 170, 64, 3]
    seq_lens = [64, 500, 2000, 3000, 64, 1300]
    cache, table, q, tok0, rows = _setup(gpu_ops, gen, lay, q_lens, seq_lens, ppb, table_order=[3, 0, 5, 1, 4, 2])
    got = _batch(gpu_ops, cache, table, q, tok0, q_lens, seq_lens, rows, ppb)
    covered = np.zeros(q.shape[0], dtype=bool)
    for i, (t, ql, sl) in enumerate(zip(tok0, q_lens, seq_lens)):
        want = _oracle(cache, q[t : t + ql], table[rows[i]], sl, ppb)
        err = assert_close(got[t : t + ql], want, what="batch seq %d (q %d over %d)" % (i, ql, sl))
        covered[t : t + ql] = True
        print("  seq %d q %d seq %d max abs err %.2e" % (i, ql, sl, err), flush=True)
    assert np.isnan(got[~covered]).all(), "rows outside every sequence were written"


def test_more_sequences_than_one_launch_equal_single_calls(gpu_ops):
    """23 sequences (three launches of at most ten) against the single-sequence entry."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(2024)
    rng = np.random.default_rng(7)
    q_lens = [int(x) for x in rng.integers(1, 90, size=23)]
    seq_lens = [ql + int(x) for ql, x in zip(q_lens, rng.integers(0, 1500, size=23))]
    cache, table, q, tok0, rows = _setup(gpu_ops, gen, lay, q_lens, seq_lens, gap=1)
    got = _batch(gpu_ops, cache, table, q, tok0, q_lens, seq_lens, rows)
    scale = 1.0 / math.sqrt(128)
    for i, (t, ql, sl) in enumerate(zip(tok0, q_lens, seq_lens)):
        one = torch.full((ql, lay.hq, 128), float("nan"), dtype=torch.float32, device=DEV)
        hip_prefill(q[t : t + ql].to(DEV), cache.views, table[i].to(device=DEV, dtype=torch.int32), sl, 1, scale,
                    out=one)
        torch.cuda.synchronize()
        assert_close(got[t : t + ql], one.cpu().numpy(), what="batch vs single, seq %d" % i)
    for i in (0, 11, 22):
        t, ql, sl = tok0[i], q_lens[i], seq_lens[i]
        assert_close(got[t : t + ql], _oracle(cache, q[t : t + ql], table[i], sl), what="batch seq %d" % i)


def test_empty_sequences_are_skipped_and_rows_checked(gpu_ops):
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(11)
    q_lens, seq_lens = [0, 5, 0], [100, 700, 0]
    cache, table, q, tok0, _ = _setup(gpu_ops, gen, lay, [1, 5, 1], [100, 700, 1])
    got = _batch(gpu_ops, cache, table, q, tok0, q_lens, seq_lens, [0, 1, 2], out_dtype=torch.float16)
    t = tok0[1]
    assert_close(got[t : t + 5], _oracle(cache, q[t : t + 5], table[1], 700), what="batch with empty sequences")
    mask = np.ones(q.shape[0], dtype=bool)
    mask[t : t + 5] = False
    assert np.isnan(got[mask]).all()
    # nothing to do at all: no launch, out untouched
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device=DEV)
    gpu_ops.prefill_paged_batch(q.to(DEV), *cache.region_args(), table.to(device=DEV, dtype=torch.int32), [], [], [],
                                [], 1, 0.1, out)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    with pytest.raises(RuntimeError, match="query longer than the KV sequence"):
        gpu_ops.prefill_paged_batch(q.to(DEV), *cache.region_args(), table.to(device=DEV, dtype=torch.int32), [0],
                                    [9], [8], [0], 1, 0.1, out)
    with pytest.raises(RuntimeError, match="sequence rows outside the query"):
        gpu_ops.prefill_paged_batch(q.to(DEV), *cache.region_args(), table.to(device=DEV, dtype=torch.int32),
                                    [q.shape[0] - 1], [2], [8], [0], 1, 0.1, out)
