"""Seeded random shapes through every entry against the oracle (GPU).

The fixed-shape tests cover the benchmark configurations and the edge cases
one at a time; this one draws a fixed, seeded set of mixed shapes -- KV heads
2 / 4, head dims 128 / 256, 1-3 pages per manager block, query lengths 1-10
(decode) and 1-700 (prefill), empty sequences, explicit split counts, up to
13 sequences in a batched prefill with block-table rows in another order --
and checks each against the float64 oracle.  Tolerance: max-abs 2e-3 with a
1e-2 relative allowance; head-dim-256 prefill uses 3e-3 absolute: its fp16
probabilities (the reference's fp16 attention keeps them in fp16 too) leave
up to 2.6e-3 on an output element near zero when a row sees few keys, the
first tokens of a chunk over an empty context (three elements past 2e-3 in
5,348 random cases, none past 2.6e-3).
"""
from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

from gpu_cases import DEV, Cache, assert_close, decode, fill_sequence, random_tables, seeded_normal
from k8v4_v030.layout import PAGE, PageLayout
from k8v4_v030.prefill import hip_prefill
from oracle import attention

pytestmark = pytest.mark.gpu

SEED = 7


def _pages(lengths, ppb):
    return sum(-(-((L + PAGE - 1) // PAGE) // ppb) for L in lengths) * ppb + 4 * ppb


def _prefill_atol(d):
    return 3e-3 if d == 256 else 2e-3


@pytest.mark.parametrize("case", range(24))
def test_random_decode(gpu_ops, case):
    rng = random.Random(SEED * 1000 + case)
    hkv, d, ppb = rng.choice([2, 4]), rng.choice([128, 256]), rng.choice([1, 1, 2, 3])
    q_len, batch = rng.randint(1, 10), rng.randint(1, 6)
    lengths = [rng.choice([0, rng.randint(q_len, 200), rng.randint(q_len, 6000)]) for _ in range(batch)]
    if max(lengths) == 0:
        lengths[0] = q_len
    splits = rng.choice([0, 0, rng.randint(batch, 300)])
    print("decode case %d hkv=%d d=%d ppb=%d q=%d lens=%s splits=%d" % (case, hkv, d, ppb, q_len, lengths, splits),
          flush=True)
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(SEED * 1000 + case)
    pages = _pages(lengths, ppb)
    table = random_tables(gen, lengths, pages, ppb=ppb)
    cache = Cache(pages, lay)
    for b, L in enumerate(lengths):
        if L:
            fill_sequence(gpu_ops, cache, gen, table[b], L, ppb=ppb)
    seq = torch.tensor(lengths, dtype=torch.int32)
    q = seeded_normal(gen, (batch * q_len, lay.hq, d))
    got = decode(gpu_ops, cache, q, table, seq, q_len, ppb=ppb, num_splits=splits).float().cpu().numpy()
    want = attention.decode_attention(q.float().numpy(), cache.blob(), cache.geom, table.numpy(), seq.numpy(), q_len,
                                      ppb, None)
    assert_close(got, want, what="random decode %d" % case)


@pytest.mark.parametrize("case", range(12))
def test_random_prefill(gpu_ops, case):
    rng = random.Random(SEED * 2000 + case)
    hkv, d, ppb = rng.choice([2, 4]), rng.choice([128, 256]), rng.choice([1, 1, 2, 3])
    q_len = rng.choice([rng.randint(1, 64), rng.randint(1, 300), rng.randint(100, 700)])
    seq_len = q_len + rng.choice([0, rng.randint(0, 500), rng.randint(0, 9000)])
    print("prefill case %d hkv=%d d=%d ppb=%d q=%d seq=%d" % (case, hkv, d, ppb, q_len, seq_len), flush=True)
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(SEED * 2000 + case)
    pages = _pages([seq_len], ppb)
    table = random_tables(gen, [seq_len], pages, ppb=ppb)
    cache = Cache(pages, lay)
    fill_sequence(gpu_ops, cache, gen, table[0], seq_len, ppb=ppb)
    q = seeded_normal(gen, (q_len, lay.hq, d))
    scale = 1.0 / math.sqrt(d)
    out = torch.full(q.shape, float("nan"), dtype=torch.float16, device=DEV)
    hip_prefill(q.to(DEV), cache.views, table[0].to(device=DEV, dtype=torch.int32), seq_len, ppb, scale, out=out)
    torch.cuda.synchronize()
    want = attention.prefill_attention(q.float().numpy(), cache.blob(), cache.geom, table[0].numpy(), seq_len, ppb,
                                       scale)
    assert_close(out.float().cpu().numpy(), want, atol=_prefill_atol(d), what="random prefill %d" % case)


@pytest.mark.parametrize("case", range(12))
def test_random_prefill_batch(gpu_ops, case):
    rng = random.Random(SEED * 3000 + case)
    hkv, d, ppb = rng.choice([2, 4]), rng.choice([128, 256]), rng.choice([1, 1, 2, 3])
    k = rng.randint(1, 13)
    q_lens = [rng.choice([0, rng.randint(1, 40), rng.randint(1, 150)]) for _ in range(k)]
    seq_lens = [ql + rng.choice([0, rng.randint(0, 300), rng.randint(0, 3000)]) for ql in q_lens]
    order = list(range(k))
    rng.shuffle(order)
    print("batch case %d hkv=%d d=%d ppb=%d q=%s seq=%s" % (case, hkv, d, ppb, q_lens, seq_lens), flush=True)
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(SEED * 3000 + case)
    lens_by_row = [0] * k
    for i, r in enumerate(order):
        lens_by_row[r] = seq_lens[i]
    pages = _pages(lens_by_row, ppb)
    table = random_tables(gen, lens_by_row, pages, ppb=ppb)
    cache = Cache(pages, lay)
    for r, L in enumerate(lens_by_row):
        if L:
            fill_sequence(gpu_ops, cache, gen, table[r], L, ppb=ppb)
    tok0, t = [], 2
    for ql in q_lens:
        tok0.append(t)
        t += ql + 1
    q = seeded_normal(gen, (t, lay.hq, d))
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device=DEV)
    scale = 1.0 / math.sqrt(d)
    gpu_ops.prefill_paged_batch(q.to(DEV), *cache.region_args(), table.to(device=DEV, dtype=torch.int32), tok0, q_lens,
                                seq_lens, order, ppb, scale, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    covered = np.zeros(t, dtype=bool)
    blob = cache.blob()
    for i in range(k):
        if q_lens[i] == 0:
            continue
        a, ql = tok0[i], q_lens[i]
        want = attention.prefill_attention(q[a:a + ql].float().numpy(), blob, cache.geom, table[order[i]].numpy(),
                                           seq_lens[i], ppb, scale)
        assert_close(got[a:a + ql], want, atol=_prefill_atol(d), what="random batch %d seq %d" % (case, i))
        covered[a:a + ql] = True
    assert np.isnan(got[~covered]).all(), "rows outside every sequence were written"
