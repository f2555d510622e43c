"""Chunked-prefill kernel vs the oracle (GPU).

The oracle (oracle/attention.py prefill_attention) is textbook bottom-right
causal softmax attention in float64 over the fp32-dequantized cache, itself
pinned to torch's scaled_dot_product_attention (tests/test_oracle.py).
Tolerance: max-abs 2e-3 with a 1e-2 relative allowance.
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


def _run(cache, q, row, seq_len, ppb=1, out_dtype=None, scale=None):
    scale = 1.0 / math.sqrt(cache.layout.head_dim) if scale is None else scale
    qd = q.to(DEV)
    out = torch.full(q.shape, float("nan"), dtype=out_dtype or q.dtype, device=DEV)
    got = hip_prefill(qd, cache.views, row.to(device=DEV, dtype=torch.int32), seq_len, ppb, scale, out=out)
    torch.cuda.synchronize()
    return got


def _oracle(cache, q, row, seq_len, ppb=1, rows=None, scale=None):
    scale = 1.0 / math.sqrt(cache.layout.head_dim) if scale is None else scale
    return attention.prefill_attention(q.float().cpu().numpy(), cache.blob(), cache.geom, row.numpy(), seq_len,
                                       ppb, scale, rows=rows)


@pytest.mark.parametrize("hkv,d,q_len,seq_len", [
    (4, 128, 1, 1), (4, 128, 7, 300), (4, 128, 64, 64), (4, 128, 100, 1000), (2, 128, 33, 2049),
    (4, 128, 250, 4000), (2, 256, 20, 500), (4, 256, 70, 700), (2, 256, 1, 129),
    # two KV heads with tile images (four or more row blocks): one launch per
    # head over its own steps, whose grid sizes the partial states
    (2, 128, 200, 300), (2, 128, 170, 3000), (2, 128, 700, 9000),
    # head dim 256 with several row blocks (converted in place: the tile
    # images pay off only for longer chunks over longer contexts)
    (2, 256, 200, 3000), (2, 256, 700, 9000), (4, 256, 90, 5000),
])
def test_prefill_matches_oracle(gpu_ops, hkv, d, q_len, seq_len):
    print("prefill hkv=%d d=%d q=%d seq=%d" % (hkv, d, q_len, seq_len), flush=True)
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(7 * q_len + seq_len + d + hkv)
    pool = (seq_len + PAGE - 1) // PAGE + 5
    table = random_tables(gen, [seq_len], pool)
    cache = Cache(pool, lay)
    fill_sequence(gpu_ops, cache, gen, table[0], seq_len)
    q = seeded_normal(gen, (q_len, lay.hq, d))
    got = _run(cache, q, table[0], seq_len).float().cpu().numpy()
    err = assert_close(got, _oracle(cache, q, table[0], seq_len), what="prefill")
    print("  max abs err %.2e" % err, flush=True)


def test_prefill_manager_blocks_and_dirty_tail(gpu_ops):
    """ppb=2 tables; the tail of the last page holds garbage codes and NaN planes."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(5)
    seq_len, q_len, ppb = 1000, 90, 2
    cache = Cache(64, lay)
    table = random_tables(gen, [seq_len], 64, ppb=ppb)
    fill_sequence(gpu_ops, cache, gen, table[0], seq_len, ppb=ppb)
    last = (seq_len - 1) // PAGE
    phys = int(table[0][last // ppb]) * ppb + last % ppb
    tail = slice(seq_len % PAGE, PAGE)
    cache.views["k"][phys, tail] = 77
    cache.views["v"][phys, tail] = 0xEE
    for plane in ("k_scale", "v_scale", "v_zero"):
        cache.views[plane][phys, tail] = float("nan")
    q = seeded_normal(gen, (q_len, 24, 128))
    got = _run(cache, q, table[0], seq_len, ppb=ppb).float().cpu().numpy()
    assert_close(got, _oracle(cache, q, table[0], seq_len, ppb=ppb), what="dirty tail")


def test_prefill_dtypes(gpu_ops):
    lay = PageLayout(2, 128)
    gen = torch.Generator().manual_seed(11)
    seq_len, q_len = 700, 50
    cache = Cache(20, lay)
    table = random_tables(gen, [seq_len], 20)
    fill_sequence(gpu_ops, cache, gen, table[0], seq_len)
    q = seeded_normal(gen, (q_len, 12, 128))
    want = _oracle(cache, q, table[0], seq_len)
    for out_dtype in (torch.float32, torch.bfloat16):
        got = _run(cache, q, table[0], seq_len, out_dtype=out_dtype)
        assert got.dtype == out_dtype
        assert_close(got.float().cpu().numpy(), want, what=str(out_dtype))
    # bf16 queries are rounded to fp16 like the reference's query.to(float16);
    # the same 2e-3 / 1e-2 holds for bf16 and fp32 outputs.
    qb = q.to(torch.bfloat16)
    want_b = _oracle(cache, qb.to(torch.float16), table[0], seq_len)
    got = _run(cache, qb, table[0], seq_len)
    assert got.dtype == torch.bfloat16
    assert_close(got.float().cpu().numpy(), want_b, what="bf16 query")
    got32 = _run(cache, qb, table[0], seq_len, out_dtype=torch.float32)
    assert assert_close(got32.cpu().numpy(), want_b, what="bf16 query, fp32 out") < 1e-3


def test_prefill_scale_is_a_parameter(gpu_ops):
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(12)
    cache = Cache(10, lay)
    table = random_tables(gen, [500], 10)
    fill_sequence(gpu_ops, cache, gen, table[0], 500)
    q = seeded_normal(gen, (40, 24, 128))
    got = _run(cache, q, table[0], 500, scale=0.05).float().cpu().numpy()
    assert_close(got, _oracle(cache, q, table[0], 500, scale=0.05), what="scale 0.05")


def test_prefill_rejections(gpu_ops):
    lay = PageLayout(4, 128)
    cache = Cache(4, lay)
    row = torch.arange(4, dtype=torch.int32)
    q = torch.zeros(10, 24, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="query longer than the KV sequence"):
        _run(cache, q, row, 9)
    with pytest.raises(RuntimeError, match=r"query has 12 heads, the K8/V4 cache holds 4 \(needs 24\)"):
        _run(cache, torch.zeros(10, 12, 128, dtype=torch.float16), row, 100)
    with pytest.raises(RuntimeError, match="block table row covers 256 tokens"):
        _run(cache, q, row, 300)
    empty = torch.zeros(0, 24, 128, dtype=torch.float16, device=DEV)
    assert hip_prefill(empty, cache.views, row.to(DEV), 5, 1, 0.1) is empty


def test_prefill_chunk_4224_over_131072_all_rows(gpu_ops):
    """The benchmark shape: a 4,224-token chunk after 131,072 cached tokens (24/4 heads, D=128).

    The chunk's own K/V are written by the store kernel first.  Every one of
    the 4,224 x 24 output rows is checked over all 135,296 keys against the
    torch restatement of the reference's prefill (oracle/torch_cpu.py, fp32
    key-tiled online softmax, itself pinned to the float64 oracle at 2e-5 in
    tests/test_oracle.py); the first and last token of each block of 256
    packed rows (row = token * 6 + head) are also checked against the float64
    oracle directly.  Tolerance: max-abs 2e-3 with a 1e-2 relative allowance."""
    from oracle import torch_cpu
    from oracle.paged import Geometry

    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(1005)
    seq_len, q_len = 131072 + 4224, 4224
    pages = seq_len // PAGE
    cache = Cache(pages + 16, lay)
    table = random_tables(gen, [seq_len], pages + 16)
    fill_sequence(gpu_ops, cache, gen, table[0], seq_len)
    q = seeded_normal(gen, (q_len, 24, 128))
    got = _run(cache, q, table[0], seq_len, out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(got).all()
    print("  all rows against the torch CPU port", flush=True)
    views = torch_cpu.region_views(torch.from_numpy(cache.blob().copy()), Geometry(4, 128))
    want_all = torch_cpu.prefill(views, q, table[0].long(), seq_len, 1.0 / math.sqrt(128)).numpy()
    err_all = assert_close(got, want_all, what="4224x131072 all rows")
    blocks = (q_len * 6 + 255) // 256
    rows = sorted({min(q_len - 1, (256 * k) // 6) for k in range(blocks)} |
                  {min(q_len - 1, (256 * k + 255) // 6) for k in range(blocks)})
    rows = np.array(rows)
    err = 0.0
    for part in np.array_split(rows, 4):
        want = _oracle(cache, q, table[0], seq_len, rows=part)
        err = max(err, assert_close(got[part], want, what="4224x131072 float64 rows"))
        # The CPU port agrees with the float64 oracle on the same rows.
        assert np.abs(want_all[part] - want).max() <= 2e-5
    print("  %d x 24 rows max abs err %.2e; %d rows vs float64 %.2e" % (q_len, err_all, rows.size, err), flush=True)


@pytest.mark.parametrize("hkv,q_len,seq_len", [(2, 1500, 7000), (4, 1400, 8000)])
def test_prefill_d256_over_tile_images_all_rows(gpu_ops, hkv, q_len, seq_len):
    """Head dim 256 with enough row blocks and pages for the per-head tile
    images (the workspace holds them: one 68 KB image per page).  Every row
    against the torch restatement of the reference's prefill, the first and
    last token of every 128-row block against the float64 oracle; max-abs
    2e-3 with a 1e-2 relative allowance."""
    from oracle import torch_cpu
    from oracle.paged import Geometry

    print("prefill d=256 tiles hkv=%d q=%d seq=%d" % (hkv, q_len, seq_len), flush=True)
    pages = -(-seq_len // PAGE)
    assert gpu_ops.prefill_workspace_bytes(seq_len, q_len, hkv, 256) > pages * 68 * 1024
    lay = PageLayout(hkv, 256)
    gen = torch.Generator().manual_seed(q_len + seq_len + hkv)
    cache = Cache(pages + 8, lay)
    table = random_tables(gen, [seq_len], pages + 8)
    fill_sequence(gpu_ops, cache, gen, table[0], seq_len)
    q = seeded_normal(gen, (q_len, lay.hq, 256))
    got = _run(cache, q, table[0], seq_len, out_dtype=torch.float32).cpu().numpy()
    views = torch_cpu.region_views(torch.from_numpy(cache.blob().copy()), Geometry(hkv, 256))
    want_all = torch_cpu.prefill(views, q, table[0].long(), seq_len, 1.0 / math.sqrt(256)).numpy()
    err_all = assert_close(got, want_all, what="d256 tiles all rows")
    blocks = (q_len * 6 + 127) // 128
    rows = np.array(sorted({min(q_len - 1, (128 * k) // 6) for k in range(blocks)} |
                           {min(q_len - 1, (128 * k + 127) // 6) for k in range(blocks)}))
    want = _oracle(cache, q, table[0], seq_len, rows=rows)
    err = assert_close(got[rows], want, what="d256 tiles float64 rows")
    print("  all rows %.2e, %d rows vs float64 %.2e" % (err_all, rows.size, err), flush=True)


@pytest.mark.parametrize("q_len,seq_len", [(3, 5000), (1, 64), (40, 40), (500, 9000)])
def test_prefill_blocks_split_across_many_work_groups(gpu_ops, q_len, seq_len):
    """Short chunks over long contexts: the balanced schedule cuts one row block into
    many pieces (down to single pages, some with no visible key for early rows)
    that the merge kernel combines."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(q_len + seq_len)
    pool = (seq_len + PAGE - 1) // PAGE + 3
    table = random_tables(gen, [seq_len], pool)
    cache = Cache(pool, lay)
    fill_sequence(gpu_ops, cache, gen, table[0], seq_len)
    q = seeded_normal(gen, (q_len, 24, 128))
    got = _run(cache, q, table[0], seq_len).float().cpu().numpy()
    assert_close(got, _oracle(cache, q, table[0], seq_len), what="split blocks")
    assert gpu_ops.prefill_workspace_bytes(seq_len, q_len, 4, 128) > 0


@pytest.mark.parametrize("d,q_len", [(128, 40), (128, 200), (256, 40)])
def test_prefill_values_near_the_fp16_limit(gpu_ops, d, q_len):
    """Every 7th token's V row alternates 60000 / -65504 (its -65504 codes
    dequantize to -8 * 125504 / 15 = -66935, beyond fp16) and its K row draws
    almost all of the softmax weight, so outputs exceed 65504 in magnitude:
    the dequantized tiles and the accumulation must stay finite and match the
    oracle for fp32 output (200 query tokens take the path that dequantizes
    each page once per head, 40 the in-kernel conversion)."""
    print("prefill large V d=%d q_len=%d" % (d, q_len), flush=True)
    lay = PageLayout(2, d)
    cache = Cache(64, lay)
    gen = torch.Generator().manual_seed(43)
    L = 3000
    table = random_tables(gen, [L], 64)
    t = torch.arange(L)
    slots = (table[0].long()[t // PAGE] * PAGE + t % PAGE).to(DEV)
    k = seeded_normal(gen, (L, 2, d))
    v = seeded_normal(gen, (L, 2, d))
    k[::7] = 4.0
    v[::7, :, 0::2] = 60000.0
    v[::7, :, 1::2] = -65504.0
    cache.store(gpu_ops, k.to(DEV), v.to(DEV), slots)
    q = seeded_normal(gen, (q_len, 12, d)).abs()
    want = _oracle(cache, q, table[0], L)
    assert np.abs(want).max() > 65504.0
    got = _run(cache, q, table[0], L, out_dtype=torch.float32)
    assert_close(got.cpu().numpy(), want, what="large V d=%d" % d)


def test_reference_named_entry_points(gpu_ops):
    """eager_prefill / head_major_prefill under the reference's module names run the same kernel."""
    from k8v4_v030.dequant import eager_prefill
    from k8v4_v030.onednn_prefill import head_major_prefill

    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(31)
    table = random_tables(gen, [700], 16)
    cache = Cache(16, lay)
    fill_sequence(gpu_ops, cache, gen, table[0], 700)
    q = seeded_normal(gen, (45, 24, 128))
    row = table[0].to(device=DEV, dtype=torch.int32)
    scale = 1.0 / math.sqrt(128)
    want = _oracle(cache, q, table[0], 700)
    for entry in (eager_prefill, head_major_prefill):
        got = entry(q.to(DEV), cache.views, row, 700, 1, scale)
        torch.cuda.synchronize()
        assert got.dtype == torch.float16 and tuple(got.shape) == (45, 24, 128)
        assert_close(got.float().cpu().numpy(), want, what=entry.__name__)
