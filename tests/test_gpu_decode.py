"""Paged decode / MTP-verify kernel vs the oracle (GPU).

Mirrors the reference's XPU regression suite (k8v4_v030/tests/test_kernel_xpu.py):
partial pages and dirty tails, prefix copy-on-write, MTP-7 == serial q=1,
builtin == explicit visible lengths, the int16 length wrap, manager-block
tables and padded tables, and an 8-sequence batch in permuted order -- plus
direct oracle parity (max-abs 2e-3 / rel 1e-2) at the benchmark shapes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_cases import DEV, Cache, assert_close, decode, fill_sequence, max_abs, random_tables, seeded_normal
from k8v4_v030.layout import PAGE, PageLayout, as_int16, block_byte_span, pages_per_block, visible_lens
from oracle import attention

pytestmark = pytest.mark.gpu


def _oracle(cache, q, table, seq_lens, q_len, ppb=1, visible=None):
    return attention.decode_attention(q.float().cpu().numpy(), cache.blob(), cache.geom, table.numpy(),
                                      seq_lens.numpy(), q_len, ppb,
                                      None if visible is None else visible.numpy())


@pytest.mark.parametrize("hkv,d,q_len", [(4, 128, 7), (4, 128, 1), (2, 128, 3), (4, 128, 10),
                                         (2, 256, 7), (4, 256, 1), (2, 256, 2), (4, 256, 5), (2, 256, 9),
                                         (4, 256, 10)])
def test_decode_matches_oracle_small(gpu_ops, hkv, d, q_len):
    print("decode small hkv=%d d=%d q=%d" % (hkv, d, q_len), flush=True)
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(100 + 10 * hkv + q_len + d)
    lengths = [1, 63, 64, 65, 130, 700, 2000]
    table = random_tables(gen, lengths, 64, width=40)
    cache = Cache(64, lay)
    for b, L in enumerate(lengths):
        fill_sequence(gpu_ops, cache, gen, table[b], L)
    seq = torch.tensor(lengths, dtype=torch.int32)
    q = seeded_normal(gen, (len(lengths) * q_len, lay.hq, d))
    got = decode(gpu_ops, cache, q, table, seq, q_len).float().cpu().numpy()
    want = _oracle(cache, q, table, seq, q_len)
    err = assert_close(got, want, what="small")
    print("  max abs err %.2e" % err, flush=True)


@pytest.mark.parametrize("hkv,q_len", [(4, 9), (2, 10)])
def test_row_split_handles_odd_chunk_counts_tiny_splits_and_visible_ends(gpu_ops, hkv, q_len):
    """Four row tiles (q_len 9-10) at 128 dims run split by rows: both waves
    of a head multiply every chunk, each chunk in the ring of the wave that
    loaded it.  Lengths with odd chunk counts, a one-chunk split, pages of
    two 64-token halves, a 33-page manager block, explicit visible ends out
    of order, and split counts from the default down to single pages."""
    print("row split hkv=%d q=%d" % (hkv, q_len), flush=True)
    lay = PageLayout(hkv, 128)
    gen = torch.Generator().manual_seed(900 + 10 * hkv + q_len)
    lengths = [1, 31, 32, 33, 95, 2113, 4097]
    ppb = 3
    table = random_tables(gen, lengths, 150, ppb=ppb)
    cache = Cache(150, lay)
    for b, L in enumerate(lengths):
        fill_sequence(gpu_ops, cache, gen, table[b], L, ppb=ppb)
    seq = torch.tensor(lengths, dtype=torch.int32)
    q = seeded_normal(gen, (len(lengths) * q_len, lay.hq, 128))
    want = _oracle(cache, q, table, seq, q_len, ppb=ppb)
    for splits in (0, 7, 80):
        got = decode(gpu_ops, cache, q, table, seq, q_len, ppb=ppb, num_splits=splits).float().cpu().numpy()
        assert_close(got, want, what="row split, %d splits" % splits)
    # Explicit ends out of causal order (tree verification): every row of a
    # token sees its own count of keys, down to one.
    vis = torch.zeros((len(lengths), 1 + q_len), dtype=torch.int32)
    for b, L in enumerate(lengths):
        vis[b, 0] = L
        ends = torch.randint(1, L + 1, (q_len,), generator=gen, dtype=torch.int32)
        vis[b, 1:] = ends
    got = decode(gpu_ops, cache, q, table, seq, q_len, ppb=ppb, visible=vis).float().cpu().numpy()
    assert_close(got, _oracle(cache, q, table, seq, q_len, ppb=ppb, visible=vis), what="row split, explicit ends")


def test_decode_config1_exact_shape(gpu_ops):
    """1 sequence, context 2,048, q=1, 24/4 heads, D=128, table = randperm(64)[:32]."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(1001)
    table = torch.randperm(64, generator=gen)[:32].to(torch.int32).view(1, 32)
    cache = Cache(64, lay)
    fill_sequence(gpu_ops, cache, gen, table[0], 2048)
    q = seeded_normal(gen, (1, 24, 128))
    seq = torch.tensor([2048], dtype=torch.int32)
    got = decode(gpu_ops, cache, q, table, seq, 1).float().cpu().numpy()
    assert_close(got, _oracle(cache, q, table, seq, 1), what="config1")


def test_decode_config3_mtp_verify(gpu_ops):
    """4 sequences x 8,192 context, 7 query tokens, random non-contiguous tables."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(1003)
    lengths = [8192] * 4
    table = random_tables(gen, lengths, 1024)
    cache = Cache(1024, lay)
    for b, L in enumerate(lengths):
        fill_sequence(gpu_ops, cache, gen, table[b], L)
    q = seeded_normal(gen, (4 * 7, 24, 128))
    seq = torch.tensor(lengths, dtype=torch.int32)
    got = decode(gpu_ops, cache, q, table, seq, 7).float().cpu().numpy()
    err = assert_close(got, _oracle(cache, q, table, seq, 7), what="config3")
    print("config3 max abs err %.2e" % err, flush=True)


def test_decode_config4_mixed_long_shared_prefix(gpu_ops):
    """Contexts {2,048; 32,768; 131,072; 200,000}, q=7, first 1,024 pages shared."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(1004)
    lengths = [2048, 32768, 131072, 200000]
    pages = [(L + 63) // 64 for L in lengths]
    shared = 1024
    unique = shared + sum(max(0, p - shared) for p in pages)
    perm = torch.randperm(unique, generator=gen).to(torch.int32)
    table = torch.zeros((4, max(pages)), dtype=torch.int32)
    cur = shared
    for b, p in enumerate(pages):
        table[b, : min(p, shared)] = perm[: min(p, shared)]
        if p > shared:
            table[b, shared:p] = perm[cur : cur + p - shared]
            cur += p - shared
    cache = Cache(unique, lay)
    print("config4: filling %d pages" % unique, flush=True)
    # The longest sequence writes the shared prefix once; the others reuse it.
    order = sorted(range(4), key=lambda b: -lengths[b])
    fill_sequence(gpu_ops, cache, gen, table[order[0]], lengths[order[0]])
    for b in order[1:]:
        if pages[b] > shared:
            fill_sequence(gpu_ops, cache, gen, table[b], lengths[b], start=shared * 64)
    q = seeded_normal(gen, (4 * 7, 24, 128))
    seq = torch.tensor(lengths, dtype=torch.int32)
    got = decode(gpu_ops, cache, q, table, seq, 7).float().cpu().numpy()
    print("config4: oracle", flush=True)
    err = assert_close(got, _oracle(cache, q, table, seq, 7), what="config4")
    print("config4 max abs err %.2e" % err, flush=True)


def test_decode_headline_shape(gpu_ops):
    """The benchmark step itself: 4 sequences x 131,072 cached tokens, 7 query
    tokens each, 24 Q / 4 KV heads, D = 128, random non-contiguous tables over
    an 8,192-page pool; all 168 output rows per head against the oracle."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(1006)
    lengths = [131072] * 4
    table = random_tables(gen, lengths, 8192)
    cache = Cache(8192, lay)
    for b, L in enumerate(lengths):
        fill_sequence(gpu_ops, cache, gen, table[b], L)
    q = seeded_normal(gen, (4 * 7, 24, 128))
    seq = torch.tensor(lengths, dtype=torch.int32)
    got = decode(gpu_ops, cache, q, table, seq, 7, out_dtype=torch.float32).cpu().numpy()
    print("headline: oracle", flush=True)
    err = assert_close(got, _oracle(cache, q, table, seq, 7), what="headline")
    print("headline max abs err %.2e" % err, flush=True)


@pytest.mark.parametrize("hkv", [2, 4])
def test_partial_pages_negative_slots_and_dirty_tail(gpu_ops, hkv):
    lay = PageLayout(hkv, 128)
    cache = Cache(4, lay)
    gen = torch.Generator().manual_seed(7)
    key = seeded_normal(gen, (130, hkv, 128)).to(DEV)
    value = seeded_normal(gen, (130, hkv, 128)).to(DEV)
    slots = torch.arange(130, dtype=torch.int64, device=DEV)
    slots[1] = -1
    cache.store(gpu_ops, key, value, slots)
    assert int(cache.views["k"][0, 1].abs().sum()) == 0
    table = torch.arange(4, dtype=torch.int32).view(1, 4)

    def run(L):
        q = key[L - 1 : L].repeat_interleave(6, dim=1)
        return decode(gpu_ops, cache, q, table, torch.tensor([L]), 1)

    for L in (63, 64, 65, 127, 129):
        out = run(L)
        assert torch.isfinite(out).all() and float(out.abs().max()) > 0
        q = key[L - 1 : L].repeat_interleave(6, dim=1)
        assert_close(out.float().cpu().numpy(), _oracle(cache, q.cpu(), table, torch.tensor([L]), 1), what="L=%d" % L)
    before, seen = run(108), run(109)
    huge = torch.full((1, hkv, 128), 50.0, dtype=torch.float16, device=DEV)
    cache.store(gpu_ops, huge, huge, torch.tensor([108], dtype=torch.int64, device=DEV))
    masked, included = run(108), run(109)
    assert max_abs(masked, before) < 1e-4
    assert max_abs(included, seen) > 1e-3


def test_unwritten_tail_with_nan_planes_is_masked(gpu_ops):
    """Rows past seq_len hold NaN scale planes; they must not reach the output."""
    lay = PageLayout(4, 128)
    cache = Cache(2, lay)
    cache.raw.view(torch.uint8).fill_(0xFF)  # every float plane is NaN
    gen = torch.Generator().manual_seed(8)
    fill_sequence(gpu_ops, cache, gen, torch.tensor([0, 1]), 70)
    q = seeded_normal(gen, (7, 24, 128))
    table = torch.tensor([[0, 1]], dtype=torch.int32)
    got = decode(gpu_ops, cache, q, table, torch.tensor([70]), 7)
    assert torch.isfinite(got).all()
    assert_close(got.float().cpu().numpy(), _oracle(cache, q, table, torch.tensor([70]), 7), what="nan tail")


@pytest.mark.parametrize("hkv", [2, 4])
def test_prefix_cow_matches_source_and_mutation_diverges(gpu_ops, hkv):
    lay = PageLayout(hkv, 128)
    block_size = 2112
    ratio = pages_per_block(block_size)
    cache = Cache(2 * ratio, lay)
    gen = torch.Generator().manual_seed(2112)
    ntok = 60
    key = seeded_normal(gen, (ntok, hkv, 128)).to(DEV)
    value = seeded_normal(gen, (ntok, hkv, 128)).to(DEV)
    cache.store(gpu_ops, key, value, torch.arange(ratio * PAGE, ratio * PAGE + ntok, device=DEV))
    q = key[-1:].repeat_interleave(6, dim=1)
    seq = torch.tensor([ntok])
    src_out = decode(gpu_ops, cache, q, torch.tensor([[1]]), seq, 1, ppb=ratio)
    before = decode(gpu_ops, cache, q, torch.tensor([[0]]), seq, 1, ppb=ratio)
    assert max_abs(src_out, before) > 1e-3
    src, nbytes = block_byte_span(1, block_size, lay)
    dst, _ = block_byte_span(0, block_size, lay)
    cache.raw[dst : dst + nbytes].copy_(cache.raw[src : src + nbytes])
    copied = decode(gpu_ops, cache, q, torch.tensor([[0]]), seq, 1, ppb=ratio)
    assert max_abs(src_out, copied) == 0.0
    cache.views["v_scale"][0, ntok - 1] *= 2.0
    mutated = decode(gpu_ops, cache, q, torch.tensor([[0]]), seq, 1, ppb=ratio)
    assert torch.isfinite(mutated).all() and max_abs(src_out, mutated) > 1e-3


# The reference's MTP-7 regression corpus (test_kernel_xpu.py:431-536) at its
# own shape (D = 256, 2 or 4 KV heads, 2,112-token manager blocks = 33 pages)
# and at the benchmark shape (D = 128, 4 KV heads).
MTP_CORPUS = [(2, 256, 59500, 33), (2, 256, 59527, 33), (2, 256, 63932, 33), (2, 256, 70000, 33),
              (4, 256, 59527, 33), (4, 256, 70000, 33), (4, 128, 59500, 26), (4, 128, 70000, 26)]


@pytest.mark.parametrize("hkv,d,seq_len,ratio", MTP_CORPUS)
def test_mtp7_long_properties(gpu_ops, hkv, d, seq_len, ratio):
    """MTP-7 == serial q=1, builtin == explicit lengths, int16 wrap differs,
    manager-block tables and padded tables agree (test_kernel_xpu.py:431-536)."""
    print("mtp7 hkv=%d d=%d L=%d" % (hkv, d, seq_len), flush=True)
    lay = PageLayout(hkv, d)
    q_len = 7
    n_pages = (seq_len + 63) // 64
    cache = Cache(n_pages, lay)
    gen = torch.Generator().manual_seed(seq_len + d + hkv)
    identity = torch.arange(n_pages, dtype=torch.int32).view(1, -1)
    fill_sequence(gpu_ops, cache, gen, identity[0], seq_len)
    q = seeded_normal(gen, (q_len, lay.hq, d))
    seq = torch.tensor([seq_len])
    parallel = decode(gpu_ops, cache, q, identity, seq, q_len)
    assert torch.isfinite(parallel).all() and float(parallel.abs().max()) > 0
    serial = torch.cat([decode(gpu_ops, cache, q[j : j + 1], identity, torch.tensor([seq_len - (q_len - 1 - j)]), 1)
                        for j in range(q_len)])
    assert max_abs(parallel, serial) < 1e-3
    vis = torch.tensor(visible_lens(seq_len, q_len), dtype=torch.int32).view(1, -1)
    assert max_abs(parallel, decode(gpu_ops, cache, q, identity, seq, q_len, visible=vis)) < 1e-3
    wrapped = decode(gpu_ops, cache, q, identity, torch.tensor([as_int16(seq_len)]), q_len)
    assert max_abs(parallel, wrapped) > 1e-2
    blocks = torch.arange(-(-n_pages // ratio), dtype=torch.int32).view(1, -1)
    assert max_abs(parallel, decode(gpu_ops, cache, q, blocks, seq, q_len, ppb=ratio)) < 1e-3
    wide = torch.cat([identity, torch.zeros(1, 4, dtype=torch.int32)], dim=1)
    assert max_abs(parallel, decode(gpu_ops, cache, q, wide, seq, q_len)) < 1e-3
    assert_close(parallel.float().cpu().numpy(), _oracle(cache, q, identity, seq, q_len), what="mtp %d" % seq_len)


@pytest.mark.parametrize("hkv,d", [(4, 128), (2, 256), (4, 256)])
def test_batch_of_eight_matches_per_sequence(gpu_ops, hkv, d):
    """The reference's 8-sequence batch (test_kernel_xpu.py:538-611), rows in
    permuted order: batched == each sequence alone, and the oracle."""
    print("batch8 hkv=%d d=%d" % (hkv, d), flush=True)
    lay = PageLayout(hkv, d)
    q_len = 7
    lengths = [70000, 128, 512, 4096, 20000, 40000, 35000, 23333]
    order = [1, 2, 4, 0, 6, 3, 7, 5]
    gen = torch.Generator().manual_seed(88 + d + hkv)
    pages = [(L + 63) // 64 for L in lengths]
    cache = Cache(sum(pages), lay)
    tables, queries, singles = [], [], []
    off = 0
    for b, L in enumerate(lengths):
        row = torch.arange(off, off + pages[b], dtype=torch.int32)
        off += pages[b]
        fill_sequence(gpu_ops, cache, gen, row, L)
        qb = seeded_normal(gen, (q_len, lay.hq, d))
        singles.append(decode(gpu_ops, cache, qb, row.view(1, -1), torch.tensor([L]), q_len))
        tables.append(row)
        queries.append(qb)
    width = max(pages)
    bt = torch.zeros((8, width), dtype=torch.int32)
    qcat = torch.empty((8 * q_len, lay.hq, d), dtype=torch.float16)
    lens = []
    for r, src in enumerate(order):
        bt[r, : pages[src]] = tables[src]
        qcat[r * q_len : (r + 1) * q_len] = queries[src]
        lens.append(lengths[src])
    batched = decode(gpu_ops, cache, qcat, bt, torch.tensor(lens), q_len)
    for r, src in enumerate(order):
        assert max_abs(batched[r * q_len : (r + 1) * q_len], singles[src]) < 1e-3, (r, lens[r])
    assert_close(batched.float().cpu().numpy(), _oracle(cache, qcat, bt, torch.tensor(lens), q_len), what="batch8")


@pytest.mark.parametrize("num_splits", [0, 70, 101])
def test_batch_beyond_one_wave(gpu_ops, num_splits):
    """70 ragged sequences (some empty): the split plan and the merge walk the
    lengths 64 at a time; default grid, one split per sequence (grid = batch)
    and an odd grid."""
    print("batch 70, splits %d" % num_splits, flush=True)
    lay = PageLayout(2, 128)
    q_len = 2
    gen = torch.Generator().manual_seed(70 + num_splits)
    lengths = torch.randint(q_len, 3000, (70,), generator=gen)
    lengths[[5, 33, 64, 69]] = 0
    pages = [(int(L) + 63) // 64 for L in lengths]
    cache = Cache(sum(pages) + 1, lay)
    bt = torch.zeros((70, max(pages)), dtype=torch.int32)
    off = 0
    for b, L in enumerate(lengths.tolist()):
        bt[b, : pages[b]] = torch.arange(off, off + pages[b], dtype=torch.int32)
        off += pages[b]
        if L:
            fill_sequence(gpu_ops, cache, gen, bt[b], L)
    q = seeded_normal(gen, (70 * q_len, 12, 128))
    out = decode(gpu_ops, cache, q, bt, lengths, q_len, out_dtype=torch.float32, num_splits=num_splits)
    assert_close(out.cpu().numpy(), _oracle(cache, q, bt, lengths, q_len), what="batch 70")


def test_explicit_visible_ends_out_of_order(gpu_ops):
    """visible_lens rows [max_end, end_0 .. end_{q-1}] that are not the causal
    staircase (tree-verify style: ends out of order, down to a single key)."""
    lay = PageLayout(4, 128)
    q_len = 5
    lens = [5000, 2300]
    vis_rows = [[4999, 4990, 3000, 4999, 1, 2500], [2300, 64, 2300, 1777, 65, 2]]
    gen = torch.Generator().manual_seed(5005)
    table = random_tables(gen, lens, 130)
    cache = Cache(130, lay)
    for b, L in enumerate(lens):
        fill_sequence(gpu_ops, cache, gen, table[b], L)
    q = seeded_normal(gen, (2 * q_len, 24, 128))
    seq = torch.tensor(lens)
    vis = torch.tensor(vis_rows, dtype=torch.int32)
    out = decode(gpu_ops, cache, q, table, seq, q_len, visible=vis, out_dtype=torch.float32)
    assert_close(out.cpu().numpy(), _oracle(cache, q, table, seq, q_len, visible=vis), what="explicit ends")


@pytest.mark.parametrize("hkv,d", [(4, 128), (2, 256), (4, 256)])
def test_zero_length_rows_and_output_dtypes(gpu_ops, hkv, d):
    print("zero-length rows hkv=%d d=%d" % (hkv, d), flush=True)
    lay = PageLayout(hkv, d)
    cache = Cache(8, lay)
    gen = torch.Generator().manual_seed(12)
    table = torch.tensor([[0, 1, 2], [3, 4, 5]], dtype=torch.int32)
    fill_sequence(gpu_ops, cache, gen, table[1], 150)
    q = seeded_normal(gen, (2 * 3, 6 * hkv, d))
    seq = torch.tensor([0, 150])
    out16 = decode(gpu_ops, cache, q, table, seq, 3)
    assert bool((out16[:3] == 0).all())
    want = _oracle(cache, q, table, seq, 3)
    out32 = decode(gpu_ops, cache, q, table, seq, 3, out_dtype=torch.float32)
    assert_close(out32.cpu().numpy(), want, what="fp32 out")
    # bf16 Q is quantized from its own (rounded) values: compare against that
    # oracle, at the same 2e-3 / 1e-2 (a bf16 output adds at most 2^-9
    # relative rounding, inside the relative allowance; the fp32 output shows
    # the kernel's own error).
    want_bf = _oracle(cache, q.to(torch.bfloat16), table, seq, 3)
    outbf = decode(gpu_ops, cache, q.to(torch.bfloat16), table, seq, 3, out_dtype=torch.bfloat16)
    assert_close(outbf.float().cpu().numpy(), want_bf, what="bf16 out")
    outbf32 = decode(gpu_ops, cache, q.to(torch.bfloat16), table, seq, 3, out_dtype=torch.float32)
    assert assert_close(outbf32.cpu().numpy(), want_bf, what="bf16 q, fp32 out") < 5e-4


@pytest.mark.parametrize("hkv,d", [(4, 128), (2, 256), (4, 256)])
def test_values_near_the_fp16_limit_survive_the_split_states(gpu_ops, hkv, d):
    """Every 7th token's V row alternates 60000 / -65504, whose -65504 codes
    dequantize beyond the fp16 range (-8 * 125504 / 15 = -66935), and its K row draws
    almost all of the softmax weight: the outputs exceed 65504 in magnitude.
    The split states (fp16, a quarter of each split's normalized output) and
    their merge must stay finite and match the oracle for fp32 output."""
    print("large V hkv=%d d=%d" % (hkv, d), flush=True)
    lay = PageLayout(hkv, d)
    cache = Cache(64, lay)
    gen = torch.Generator().manual_seed(41)
    table = random_tables(gen, [3000], 64)
    L = 3000
    t = torch.arange(L)
    slots = (table[0].long()[t // PAGE] * PAGE + t % PAGE).to(DEV)
    k = seeded_normal(gen, (L, hkv, d))
    v = seeded_normal(gen, (L, hkv, d))
    k[::7] = 4.0
    v[::7, :, 0::2] = 60000.0
    v[::7, :, 1::2] = -65504.0
    cache.store(gpu_ops, k.to(DEV), v.to(DEV), slots)
    q = seeded_normal(gen, (3, 6 * hkv, d)).abs()
    seq = torch.tensor([L])
    want = _oracle(cache, q, table, seq, 3)
    assert np.abs(want).max() > 65504.0
    for splits in (0, 23):
        out = decode(gpu_ops, cache, q, table, seq, 3, out_dtype=torch.float32, num_splits=splits)
        assert_close(out.cpu().numpy(), want, what="large V, %d splits" % splits)


def test_split_count_does_not_change_the_answer(gpu_ops):
    lay = PageLayout(4, 128)
    cache = Cache(300, lay)
    gen = torch.Generator().manual_seed(31)
    table = random_tables(gen, [9000, 5000], 300)
    for b, L in enumerate([9000, 5000]):
        fill_sequence(gpu_ops, cache, gen, table[b], L)
    q = seeded_normal(gen, (14, 24, 128))
    seq = torch.tensor([9000, 5000])
    outs = [decode(gpu_ops, cache, q, table, seq, 7, num_splits=s) for s in (2, 3, 17, 64, 0)]
    for o in outs[1:]:
        assert max_abs(o, outs[0]) < 1e-3


def test_rejects_bad_heads_and_q_len(gpu_ops):
    lay = PageLayout(2, 128)
    cache = Cache(4, lay)
    table = torch.arange(4, dtype=torch.int32).view(1, 4)
    for hkv in (3, 8, 1):
        q = torch.randn(1, 6 * hkv, 128, dtype=torch.float16)
        with pytest.raises(RuntimeError, match=r"unsupported per-GPU KV head count %d \(this library serves 2 or 4\)" % hkv):
            decode(gpu_ops, cache, q, table, torch.tensor([4]), 1)
    q = torch.randn(11, 12, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="q_len"):
        decode(gpu_ops, cache, q, table, torch.tensor([40]), 11)


def test_graph_capture_replays_with_new_lengths(gpu_ops):
    """The op is capturable: replays read the device-resident lengths each time."""
    lay = PageLayout(4, 128)
    cache = Cache(200, lay)
    gen = torch.Generator().manual_seed(41)
    table = random_tables(gen, [6000, 6000], 200).to(DEV)
    for b in range(2):
        fill_sequence(gpu_ops, cache, gen, table[b].cpu(), 6000)
    q = seeded_normal(gen, (14, 24, 128)).to(DEV)
    seq = torch.tensor([6000, 6000], dtype=torch.int32, device=DEV)
    nbytes = gpu_ops.attn_workspace_bytes(2, table.shape[1], 1, 7, 4, 128)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=DEV)
    out = torch.zeros(q.shape, dtype=torch.float16, device=DEV)
    args = (q, None, None, *cache.region_args(), table, seq, None, ws, None, None, None, out, 7, 1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gpu_ops.int8k_int4v_attn_batch(*args)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gpu_ops.int8k_int4v_attn_batch(*args)
    for lens in ([6000, 6000], [100, 5999], [4097, 1], [6000, 64]):
        seq.copy_(torch.tensor(lens, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = decode(gpu_ops, cache, q.cpu(), table.cpu(), torch.tensor(lens), 7)
        assert max_abs(replayed, eager) == 0.0, lens


def test_bound_call_and_stages_match_the_plain_op(gpu_ops):
    """bind_* launches the same kernels; stages 1 then 2 equal stages 3, bit for bit."""
    lay = PageLayout(4, 128)
    cache = Cache(300, lay)
    gen = torch.Generator().manual_seed(53)
    table = random_tables(gen, [9000, 3000], 300)
    for b, L in enumerate([9000, 3000]):
        fill_sequence(gpu_ops, cache, gen, table[b], L)
    q = seeded_normal(gen, (14, 24, 128))
    seq = torch.tensor([9000, 3000])
    plain = decode(gpu_ops, cache, q, table, seq, 7)
    bt, sl, qd = table.to(DEV), seq.to(device=DEV, dtype=torch.int32), q.to(DEV)
    nbytes = gpu_ops.attn_workspace_bytes(2, bt.shape[1], 1, 7, 4, 128)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=DEV)
    out = torch.full(q.shape, float("nan"), dtype=torch.float16, device=DEV)
    call = gpu_ops.bind_int8k_int4v_attn_batch(qd, None, None, *cache.region_args(), bt, sl, None, ws,
                                               None, None, None, out, 7, 1)
    call()
    torch.cuda.synchronize()
    assert max_abs(out, plain) == 0.0
    out.fill_(float("nan"))
    call(stages=1)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all(), "split-only stage wrote the output"
    call(stages=2)
    torch.cuda.synchronize()
    assert max_abs(out, plain) == 0.0
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()  # creates the event handle
    out.fill_(float("nan"))
    call(split_done_event=ev.cuda_event)
    torch.cuda.synchronize()
    assert max_abs(out, plain) == 0.0
    # New lengths in the same storage are read at launch time.
    sl.copy_(torch.tensor([2500, 1000], dtype=torch.int32))
    call()
    torch.cuda.synchronize()
    again = decode(gpu_ops, cache, q, table, torch.tensor([2500, 1000]), 7)
    assert max_abs(out, again) == 0.0
    with pytest.raises(RuntimeError, match="stages"):
        call(stages=0)


def test_no_in_kernel_wait_gave_up(gpu_ops):
    """Every paired-halves handshake of the decode runs above ended normally
    (a capped wait that gives up is counted on the device, and would mean a
    wrong output)."""
    from k8v4_v030 import ops_api

    torch.cuda.synchronize()
    assert ops_api.load_library().k8v4_decode_fault_count() == 0
