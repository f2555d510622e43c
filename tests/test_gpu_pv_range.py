"""P' = p * v_scale in fp16 at the edge of the V range (GPU).

Both attention kernels pack P' = p * v_scale into fp16 MFMA operands, where p
is exp2 of the score minus a lazily moved running max.  The cache below makes
p as large as the lazy rescale allows: every key's K row is c_t times a ones
vector (int8 codes all 127, k_scale = c_t / 127), with c_t rising so that each
32-token chunk scores 0.25 (log2 units) above the one before against an
all-ones query, and every V row alternates +-65504 over its dims, the widest
range fp16 allows (v_scale = 131008 / 15), with the sign of the pattern
flipped from one chunk to the next so the output depends on every chunk's
weight.  With a rescale threshold of 2^t, p reaches 2^t before the running
max moves, so P' = p * v_scale would pass 65504 for any t above 2.9; the
outputs must stay finite and match the oracle (an overflow gives inf, a
saturating conversion a wrong weight).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from gpu_cases import DEV, Cache, assert_close, decode, random_tables
from k8v4_v030.layout import PAGE, PageLayout
from k8v4_v030.prefill import hip_prefill
from oracle import attention

pytestmark = pytest.mark.gpu

# Score of a ones query against c * ones over 128 dims, in log2 units per
# unit of c: 128 * c / sqrt(128) * log2(e).
_LOG2_PER_C = 128.0 / math.sqrt(128.0) * 1.4426950408889634


def _rising_cache(gpu_ops, seq_len, seed):
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(seed)
    pool = (seq_len + PAGE - 1) // PAGE + 3
    table = random_tables(gen, [seq_len], pool)
    cache = Cache(pool, lay)
    t = torch.arange(seq_len)
    c = (t // 32).float() * (0.25 / _LOG2_PER_C)
    k = (c[:, None, None] * torch.ones((seq_len, 4, 128))).to(torch.float16)
    sign = 1.0 - 2.0 * ((t // 32) % 2).float()
    v = (sign[:, None, None] * torch.full((seq_len, 4, 128), 65504.0)).to(torch.float16)
    v[:, :, 1::2] = -v[:, :, 1::2]
    slots = (table[0].long()[t // PAGE] * PAGE + t % PAGE).to(DEV)
    cache.store(gpu_ops, k.to(DEV), v.to(DEV), slots)
    return cache, table


def test_decode_pv_stays_finite_at_the_v_range_edge(gpu_ops):
    seq_len, q_len = 2048, 1
    cache, table = _rising_cache(gpu_ops, seq_len, 51)
    q = torch.ones((q_len, 24, 128), dtype=torch.float16)
    want = attention.decode_attention(q.float().numpy(), cache.blob(), cache.geom, table.numpy(),
                                      np.array([seq_len]), q_len)
    assert np.abs(want).max() > 4.0e3
    for splits in (1, 0):  # one split: every chunk through one running max; default split count
        out = decode(gpu_ops, cache, q, table, torch.tensor([seq_len]), q_len, out_dtype=torch.float32,
                     num_splits=splits)
        assert_close(out.cpu().numpy(), want, what="decode, %d splits" % splits)


def test_prefill_pv_stays_finite_at_the_v_range_edge(gpu_ops):
    seq_len, q_len = 2048, 8
    cache, table = _rising_cache(gpu_ops, seq_len, 52)
    q = torch.ones((q_len, 24, 128), dtype=torch.float16)
    scale = 1.0 / math.sqrt(128.0)
    out = torch.full((q_len, 24, 128), float("nan"), dtype=torch.float32, device=DEV)
    hip_prefill(q.to(DEV), cache.views, table[0].to(device=DEV, dtype=torch.int32), seq_len, 1, scale, out=out)
    torch.cuda.synchronize()
    want = attention.prefill_attention(q.float().numpy(), cache.blob(), cache.geom, table[0].numpy(), seq_len, 1,
                                       scale)
    assert np.abs(want).max() > 4.0e3
    # The prefill K tile holds code * k_scale rounded to fp16 (2^-12 relative),
    # and here every row's rounding error is the same, which shifts whole
    # chunks' weights by up to ~0.3%; against outputs that cancel +-61137
    # terms down to ~5e3 that is ~1e2 absolute.  An overflowing or saturating
    # P' misweights tokens by percents to orders of magnitude: the tolerance
    # is 1% of the V magnitude.
    assert_close(out.cpu().numpy(), want, atol=611.0, rtol=1e-2, what="prefill")
