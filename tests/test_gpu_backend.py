"""vLLM backend glue on the GPU: store + decode + prefill steps through
``Xe2K8V4Impl`` against the oracle, in vLLM's own tensor shapes (the live layer
``[block, kv_head, token, slot_bytes]``, bf16 rows sliced out of a fused qkv
buffer), a mixed prefill/decode step, manager blocks of 33 pages at D = 256,
and a captured decode step replayed with new lengths.

Reference behaviour: k8v4_v030/backend.py:225-431 (do_kv_cache_update,
forward, _packed, _attn_batch, _eager); the oracle is oracle/attention.py.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from backend_cases import backend, common_metadata, make_builder, make_impl, slots_for, vllm_cache
from gpu_cases import DEV, assert_close, max_abs
from k8v4_v030.layout import PageLayout
from oracle import attention, paged

pytestmark = pytest.mark.gpu


def _blob(cache):
    torch.cuda.synchronize()
    return cache.view(torch.uint8).reshape(-1).cpu().numpy()


def _qkv(gen, ntok, lay, dtype):
    """Rows of a fused [T, (HQ + 2 HKV) * D] projection, as vLLM slices them."""
    hq, hkv, d = lay.hq, lay.hkv, lay.head_dim
    qkv = torch.randn((ntok, (hq + 2 * hkv) * d), generator=gen).to(dtype).to(DEV)
    q = qkv[:, : hq * d].unflatten(1, (hq, d))
    k = qkv[:, hq * d : (hq + hkv) * d].unflatten(1, (hkv, d))
    v = qkv[:, (hq + hkv) * d :].unflatten(1, (hkv, d))
    return q, k, v


def _fill(impl, cache, gen, table, lengths, block_tokens, lay, dtype):
    """Store every context token of every request through the backend."""
    for b, L in enumerate(lengths):
        if L == 0:
            continue
        _, k, v = _qkv(gen, L, lay, dtype)
        slots = slots_for(table[b], range(L), block_tokens).to(DEV)
        impl.do_kv_cache_update(None, k, v, cache, slots)


def _table(gen, lengths, num_blocks, block_tokens, width):
    perm = torch.randperm(num_blocks, generator=gen).to(torch.int32)
    table = torch.zeros((len(lengths), width), dtype=torch.int32)
    cur = 0
    for b, L in enumerate(lengths):
        n = -(-L // block_tokens)
        table[b, :n] = perm[cur : cur + n]
        cur += n
    return table


def test_store_through_backend_is_bit_exact():
    lay = PageLayout(4, 128)
    impl = make_impl()
    cache = vllm_cache(8, 64, lay, DEV)
    gen = torch.Generator().manual_seed(3)
    _, k, v = _qkv(gen, 300, lay, torch.bfloat16)
    slots = torch.randperm(8 * 64, generator=gen)[:300].to(torch.int64)
    impl.do_kv_cache_update(None, k, v, cache, slots.to(DEV))
    want = paged.new_blob(8, paged.Geometry(4, 128))
    paged.store(want, paged.Geometry(4, 128), k.float().cpu().numpy(), v.float().cpu().numpy(), slots.numpy())
    assert np.array_equal(_blob(cache), want)


@pytest.mark.parametrize("dtype,out_dtype", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                             (torch.bfloat16, torch.float32)])
def test_uniform_decode_step(dtype, out_dtype):
    """MTP-verify step: q = 7 for every request; one batched launch, rows in place.
    bf16 rows are checked at the same 2e-3 / 1e-2 as fp16 (a bf16 output adds at
    most 2^-9 relative rounding, inside the relative allowance); the fp32
    output shows the kernel's own error without any output rounding."""
    lay = PageLayout(4, 128)
    impl = make_impl()
    builder = make_builder(device=DEV, block_size=64, kernel_block=64)
    gen = torch.Generator().manual_seed(11)
    lengths = [300, 1000, 2051]
    table = _table(gen, lengths, 100, 64, 40)
    cache = vllm_cache(100, 64, lay, DEV)
    _fill(impl, cache, gen, table, [L - 7 for L in lengths], 64, lay, dtype)
    q, k, v = _qkv(gen, 21, lay, dtype)
    pos = [L - 7 + j for L in lengths for j in range(7)]
    req = [b for b in range(3) for _ in range(7)]
    slots = torch.stack([slots_for(table[req[i]], [pos[i]], 64)[0] for i in range(21)])
    meta = builder.build(0, common_metadata([7, 7, 7], lengths, table, slots, DEV))
    assert meta.packed_q_len == 7
    impl.do_kv_cache_update(None, k, v, cache, meta.slot_mapping)
    out = torch.full((21, 24 * 128), float("nan"), dtype=out_dtype, device=DEV)
    impl.forward(None, q, k, v, cache, meta, out)
    want = attention.decode_attention(q.float().cpu().numpy(), _blob(cache), paged.Geometry(4, 128), table.numpy(),
                                      np.array(lengths), 7)
    err = assert_close(out.view(21, 24, 128).float().cpu().numpy(), want, what="backend decode")
    if out_dtype == torch.float32:
        assert err < 5e-4, err


def test_mixed_step_runs_decode_batched_and_prefill_per_request():
    lay = PageLayout(4, 128)
    impl = make_impl()
    builder = make_builder(device=DEV)
    gen = torch.Generator().manual_seed(12)
    q_lens = [1, 1, 200, 150]
    lengths = [500, 64, 200, 1100]
    table = _table(gen, lengths, 60, 64, 20)
    cache = vllm_cache(60, 64, lay, DEV)
    _fill(impl, cache, gen, table, [L - q for L, q in zip(lengths, q_lens)], 64, lay, torch.float16)
    ntok = sum(q_lens)
    q, k, v = _qkv(gen, ntok, lay, torch.float16)
    slots = torch.cat([slots_for(table[b], range(L - ql, L), 64) for b, (L, ql) in enumerate(zip(lengths, q_lens))])
    meta = builder.build(0, common_metadata(q_lens, lengths, table, slots, DEV))
    assert meta.packed_q_len == 0
    impl.do_kv_cache_update(None, k, v, cache, meta.slot_mapping)
    out = torch.full((ntok, 24, 128), float("nan"), dtype=torch.float16, device=DEV)
    impl.forward(None, q, k, v, cache, meta, out)
    blob, geom = _blob(cache), paged.Geometry(4, 128)
    got = out.float().cpu().numpy()
    qf = q.float().cpu().numpy()
    want_dec = attention.decode_attention(qf[:2], blob, geom, table[:2].numpy(), np.array(lengths[:2]), 1)
    assert_close(got[:2], want_dec, what="decode rows")
    t0 = 2
    for b in (2, 3):
        rows = q_lens[b]
        want = attention.prefill_attention(qf[t0 : t0 + rows], blob, geom, table[b].numpy(), lengths[b], 1,
                                           1.0 / math.sqrt(128))
        assert_close(got[t0 : t0 + rows], want, what="prefill rows of request %d" % b)
        t0 += rows


def test_mixed_step_batches_the_short_prefills():
    """Decode rows, four short chunks (12 to 128 tokens: one batched prefill
    launch) and a 129-token chunk (the single entry) in one step."""
    lay = PageLayout(4, 128)
    impl = make_impl()
    builder = make_builder(device=DEV)
    gen = torch.Generator().manual_seed(21)
    q_lens = [1, 1, 30, 64, 128, 129, 12]
    lengths = [500, 64, 400, 64, 900, 1300, 77]
    table = _table(gen, lengths, 120, 64, 24)
    cache = vllm_cache(120, 64, lay, DEV)
    _fill(impl, cache, gen, table, [L - q for L, q in zip(lengths, q_lens)], 64, lay, torch.float16)
    ntok = sum(q_lens)
    q, k, v = _qkv(gen, ntok, lay, torch.float16)
    slots = torch.cat([slots_for(table[b], range(L - ql, L), 64) for b, (L, ql) in enumerate(zip(lengths, q_lens))])
    meta = builder.build(0, common_metadata(q_lens, lengths, table, slots, DEV))
    assert [s.width for s in meta.prefill_seqs] == [30, 64, 128, 129, 12]
    impl.do_kv_cache_update(None, k, v, cache, meta.slot_mapping)
    out = torch.full((ntok, 24, 128), float("nan"), dtype=torch.float16, device=DEV)
    impl.forward(None, q, k, v, cache, meta, out)
    blob, geom = _blob(cache), paged.Geometry(4, 128)
    got = out.float().cpu().numpy()
    qf = q.float().cpu().numpy()
    want_dec = attention.decode_attention(qf[:2], blob, geom, table[:2].numpy(), np.array(lengths[:2]), 1)
    assert_close(got[:2], want_dec, what="decode rows")
    t0 = 2
    for b in range(2, len(q_lens)):
        rows = q_lens[b]
        want = attention.prefill_attention(qf[t0 : t0 + rows], blob, geom, table[b].numpy(), lengths[b], 1,
                                           1.0 / math.sqrt(128))
        assert_close(got[t0 : t0 + rows], want, what="prefill rows of request %d" % b)
        t0 += rows


def test_manager_blocks_of_33_pages_at_d256():
    """The reference's deployment shape: TP2 rank (2 KV / 12 Q heads), D = 256,
    2,112-token manager blocks addressed directly (33 kernel pages per entry)."""
    lay = PageLayout(2, 256)
    impl = make_impl(hkv=2, head=256)
    builder = make_builder(hkv=2, head=256, device=DEV, block_size=2112, kernel_block=None, max_model_len=4 * 2112)
    gen = torch.Generator().manual_seed(13)
    lengths = [5000, 2200]
    table = _table(gen, lengths, 8, 2112, 4)
    cache = vllm_cache(8, 2112, lay, DEV)
    _fill(impl, cache, gen, table, [L - 3 for L in lengths], 2112, lay, torch.bfloat16)
    q, k, v = _qkv(gen, 6, lay, torch.bfloat16)
    slots = torch.cat([slots_for(table[b], range(L - 3, L), 2112) for b, L in enumerate(lengths)])
    meta = builder.build(0, common_metadata([3, 3], lengths, table, slots, DEV))
    assert meta.pages_per_block == 33 and meta.packed_q_len == 3
    impl.do_kv_cache_update(None, k, v, cache, meta.slot_mapping)
    out = torch.empty((6, 12, 256), dtype=torch.bfloat16, device=DEV)
    impl.forward(None, q, k, v, cache, meta, out)
    want = attention.decode_attention(q.float().cpu().numpy(), _blob(cache), paged.Geometry(2, 256), table.numpy(),
                                      np.array(lengths), 3, 33)
    assert_close(out.float().cpu().numpy(), want, what="ppb 33 decode")


def test_many_short_sequences_fit_the_scratch():
    """A decode batch far wider than its block table (64 sequences of at most
    4 pages, q = 7: more split states than 3 x table width x pages per entry)
    runs on the scratch the builder sized, against the oracle."""
    from k8v4_v030.scratch import clear_scratch

    clear_scratch()
    lay = PageLayout(4, 128)
    impl = make_impl()
    builder = make_builder(device=DEV, max_model_len=256, max_seqs=64, max_batched=512, capture=(64, 448))
    gen = torch.Generator().manual_seed(15)
    lengths = [int(x) for x in torch.randint(7, 257, (64,), generator=gen)]
    table = _table(gen, lengths, 4 * 64, 64, 4)
    cache = vllm_cache(4 * 64, 64, lay, DEV)
    _fill(impl, cache, gen, table, [L - 7 for L in lengths], 64, lay, torch.float16)
    q, k, v = _qkv(gen, 64 * 7, lay, torch.float16)
    slots = torch.cat([slots_for(table[b], range(L - 7, L), 64) for b, L in enumerate(lengths)])
    meta = builder.build(0, common_metadata([7] * 64, lengths, table, slots, DEV))
    impl.do_kv_cache_update(None, k, v, cache, meta.slot_mapping)
    out = torch.full((64 * 7, 24, 128), float("nan"), dtype=torch.float16, device=DEV)
    impl.forward(None, q, k, v, cache, meta, out)
    want = attention.decode_attention(q.float().cpu().numpy(), _blob(cache), paged.Geometry(4, 128), table.numpy(),
                                      np.array(lengths), 7)
    assert_close(out.float().cpu().numpy(), want, what="64 short sequences")
    clear_scratch()


def test_step_allocates_nothing_after_the_scratch():
    """A mixed step (decode run + prefill) draws every workspace from the scratch."""
    lay = PageLayout(4, 128)
    impl = make_impl()
    builder = make_builder(device=DEV)
    gen = torch.Generator().manual_seed(16)
    q_lens, lengths = [7, 7, 300, 40], [900, 700, 1500, 600]
    table = _table(gen, lengths, 60, 64, 24)
    cache = vllm_cache(60, 64, lay, DEV)
    _fill(impl, cache, gen, table, [L - q for L, q in zip(lengths, q_lens)], 64, lay, torch.float16)
    q, k, v = _qkv(gen, sum(q_lens), lay, torch.float16)
    meta = builder.build(0, common_metadata(q_lens, lengths, table, torch.zeros(sum(q_lens), dtype=torch.int64), DEV))
    out = torch.zeros((sum(q_lens), 24, 128), dtype=torch.float16, device=DEV)
    impl.forward(None, q, k, v, cache, meta, out)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    impl.forward(None, q, k, v, cache, meta, out)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before


def test_captured_decode_step_replays_with_new_lengths():
    lay = PageLayout(4, 128)
    impl = make_impl()
    builder = make_builder(device=DEV)
    gen = torch.Generator().manual_seed(14)
    lengths = [2000, 900]
    table = _table(gen, lengths, 60, 64, 32)
    cache = vllm_cache(60, 64, lay, DEV)
    _fill(impl, cache, gen, table, lengths, 64, lay, torch.bfloat16)
    q, k, v = _qkv(gen, 14, lay, torch.bfloat16)
    meta = builder.build(0, common_metadata([7, 7], lengths, table, torch.zeros(14, dtype=torch.int64), DEV))
    out = torch.zeros((14, 24, 128), dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        impl.forward(None, q, k, v, cache, meta, out)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        impl.forward(None, q, k, v, cache, meta, out)
    for lens in ([2000, 900], [1500, 64], [7, 800]):
        meta.seq_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager_meta = builder.build(0, common_metadata([7, 7], lens, table, torch.zeros(14, dtype=torch.int64), DEV))
        eager = torch.zeros_like(out)
        impl.forward(None, q, k, v, cache, eager_meta, eager)
        torch.cuda.synchronize()
        assert max_abs(replayed, eager) == 0.0, lens


def test_prefill_inside_a_graph_is_refused(monkeypatch):
    """Only the uniform decode step is capturable; a prefill step raises before
    it enqueues anything (the reference refuses XPU graphs the same way)."""
    lay = PageLayout(4, 128)
    impl = make_impl()
    builder = make_builder(device=DEV)
    cache = vllm_cache(4, 64, lay, DEV)
    table = torch.zeros((1, 4), dtype=torch.int32)
    meta = builder.build(0, common_metadata([20], [20], table, torch.zeros(20, dtype=torch.int64), DEV))
    q = torch.zeros((20, 24, 128), dtype=torch.float16, device=DEV)
    out = torch.zeros_like(q)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="prefill cannot run inside a HIP graph"):
        impl.forward(None, q, q, q, cache, meta, out)
