"""The rest of the reference op table on the GPU (k8v4_v030/native/xe2_kv_ops.cpp:1779-1822).

* ``q_quant_once`` and the token-row pack of ``int8k_int4v_s1_varlen_from_q``:
  codes and fp32 scales bit-exact to the oracle's K rule, pad rows zero;
* ``int8k_int4v_s1_paged`` (workspace owned by the library) equals the batch op
  and the oracle, for both head layouts interleaved in one process, and repeats
  bit for bit (the reference's test_kernel_xpu.py:223-293);
* ``int8k_int4v_s1_varlen_paged`` with explicit causal ends, manager blocks and
  a workspace sized the reference's way ([W * ppb * hkv, 64, D] fp32);
* ``int8k_int4v_decode_step`` (store + attend) against the oracle;
* ``k_store_paged`` + ``v_store_paged`` write exactly the bytes of ``kv_store_paged``.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_cases import DEV, Cache, assert_close, decode, fill_sequence, max_abs, random_tables, seeded_normal
from k8v4_v030.layout import GQA, PAGE, PageLayout
from oracle import attention, paged, quant

pytestmark = pytest.mark.gpu


def _tile_want(rows: np.ndarray):
    """Oracle codes and stored scales of a [hkv, 64, D] float tile."""
    codes, scale = quant.quant_k(rows)
    return codes, quant.stored_f32(scale)


@pytest.mark.parametrize("hkv,d,dtype", [(2, 256, torch.float16), (4, 128, torch.float16), (4, 256, torch.bfloat16)])
def test_q_quant_once_is_bit_exact(gpu_ops, hkv, d, dtype):
    gen = torch.Generator().manual_seed(600 + hkv + d)
    pad = (torch.randn((hkv, PAGE, d), generator=gen) * 3).to(dtype)
    pad[:, 40:] = 0  # pad rows, as the reference's callers leave them
    # exact rounding ties: x = amax * (2k + 1) / 254 for amax a multiple of 127
    pad[0, 3] = 0
    pad[0, 3, :8] = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -63.5, 63.5, -127.0], dtype=dtype)
    q8 = torch.full((hkv, PAGE, d), 77, dtype=torch.int8, device=DEV)
    qs = torch.full((hkv, PAGE), float("nan"), dtype=torch.float32, device=DEV)
    gpu_ops.q_quant_once(pad.to(DEV), q8, qs)
    codes, scales = _tile_want(pad.float().numpy())
    assert np.array_equal(q8.cpu().numpy(), codes)
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), scales.view(np.uint32))
    assert not q8[:, 40:].any() and not qs[:, 40:].any()


def test_token_rows_are_packed_into_the_tile(gpu_ops):
    """varlen_from_q packs [T, HQ, D] rows (row = token * 6 + group) and zeroes the rest."""
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(611)
    cache = Cache(8, lay)
    table = torch.arange(8, dtype=torch.int32).view(1, 8)
    fill_sequence(gpu_ops, cache, gen, table[0], 500)
    q = seeded_normal(gen, (7, 24, 128)).to(DEV)
    q8 = torch.full((4, PAGE, 128), 5, dtype=torch.int8, device=DEV)
    qs = torch.full((4, PAGE), 9.0, dtype=torch.float32, device=DEV)
    out = torch.zeros((7, 24, 128), dtype=torch.float32, device=DEV)
    gpu_ops.int8k_int4v_s1_varlen_from_q(q, q8, qs, *cache.region_args(), table.to(DEV),
                                         torch.tensor([500], dtype=torch.int32, device=DEV), None, None, None, None,
                                         None, out)
    tile = np.zeros((4, PAGE, 128))
    tile[:, :42] = q.float().cpu().numpy().reshape(7, 4, 6, 128).transpose(1, 0, 2, 3).reshape(4, 42, 128)
    codes, scales = _tile_want(tile)
    assert np.array_equal(q8.cpu().numpy(), codes)
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), scales.view(np.uint32))
    want = attention.decode_attention(q.float().cpu().numpy(), cache.blob(), cache.geom, table.numpy(), [500], 7)
    assert_close(out.cpu().numpy(), want, what="varlen_from_q")


def test_legacy_op_interleaves_both_layouts(gpu_ops):
    """q_quant_once + int8k_int4v_s1_paged (library workspace) equals the batch op
    for 2 and 4 KV heads, alternating layouts, and repeats bit for bit."""
    legacy = {}
    for rerun in (False, True):
        for hkv in (2, 4):
            lay = PageLayout(hkv, 256)
            cache = Cache(4, lay)
            gen = torch.Generator().manual_seed(5)
            key = torch.randn(200, hkv, 256, generator=gen, dtype=torch.float16).to(DEV)
            value = torch.randn(200, hkv, 256, generator=gen, dtype=torch.float16).to(DEV)
            cache.store(gpu_ops, key, value, torch.arange(200, dtype=torch.int64, device=DEV))
            query = torch.randn(1, 6 * hkv, 256, generator=gen, dtype=torch.float16).to(DEV)
            table = torch.arange(4, dtype=torch.int32, device=DEV).view(1, 4)
            seq = torch.tensor([200], dtype=torch.int32, device=DEV)
            pad = torch.zeros(hkv, PAGE, 256, dtype=torch.float16, device=DEV)
            pad[:, :GQA] = query[0].view(hkv, GQA, 256)
            q8 = torch.empty((hkv, PAGE, 256), dtype=torch.int8, device=DEV)
            qs = torch.empty((hkv, PAGE), dtype=torch.float32, device=DEV)
            gpu_ops.q_quant_once(pad, q8, qs)
            out = torch.zeros((1, 6 * hkv, 256), dtype=torch.float16, device=DEV)
            gpu_ops.int8k_int4v_s1_paged(q8, qs, *cache.region_args(), table, seq, out)
            torch.cuda.synchronize()
            if rerun:
                assert torch.equal(out, legacy[hkv]), hkv
                continue
            legacy[hkv] = out.clone()
            batch = decode(gpu_ops, cache, query.cpu(), table.cpu(), seq.cpu(), 1)
            assert max_abs(out, batch) < 1e-4
            want = attention.decode_attention(query.float().cpu().numpy(), cache.blob(), cache.geom, table.cpu().numpy(),
                                              [200], 1)
            assert_close(out.float().cpu().numpy(), want, what="legacy hkv=%d" % hkv)


def test_varlen_paged_with_visible_ends_manager_blocks_and_reference_workspace(gpu_ops):
    lay = PageLayout(2, 256)
    gen = torch.Generator().manual_seed(612)
    ppb, width, L, tq = 33, 3, 5000, 7
    cache = Cache(width * ppb * 2, lay)
    table = torch.tensor([[4, 1, 3]], dtype=torch.int32)
    fill_sequence(gpu_ops, cache, gen, table[0], L, ppb=ppb)
    q = seeded_normal(gen, (tq, 12, 256)).to(DEV)
    vis = torch.tensor([L - 3] + [L - 100 + 13 * j for j in range(tq)], dtype=torch.int32)
    q8 = torch.empty((2, PAGE, 256), dtype=torch.int8, device=DEV)
    qs = torch.empty((2, PAGE), dtype=torch.float32, device=DEV)
    nprog = width * ppb * 2  # the reference's workspace_programs
    partials = torch.empty((nprog, PAGE, 256), dtype=torch.float32, device=DEV)
    m_ws = torch.empty((nprog, PAGE), dtype=torch.float32, device=DEV)
    out = torch.full((tq, 12, 256), float("nan"), dtype=torch.float32, device=DEV)
    gpu_ops.int8k_int4v_s1_varlen_from_q(q, q8, qs, *cache.region_args(), table.to(DEV),
                                         torch.tensor([L], dtype=torch.int32, device=DEV), vis.to(DEV), partials,
                                         m_ws, m_ws, partials, out, ppb)
    want = attention.decode_attention(q.float().cpu().numpy(), cache.blob(), cache.geom, table.numpy(), [L], tq, ppb,
                                      vis.view(1, -1).numpy())
    assert_close(out.cpu().numpy(), want, what="varlen ppb 33 visible ends")
    # the same tile through int8k_int4v_s1_varlen_paged directly
    again = torch.full_like(out, float("nan"))
    gpu_ops.int8k_int4v_s1_varlen_paged(q8, qs, *cache.region_args(), table.to(DEV),
                                        torch.tensor([L], dtype=torch.int32, device=DEV), vis.to(DEV), partials, m_ws,
                                        m_ws, partials, again, ppb)
    torch.cuda.synchronize()
    assert torch.equal(out, again)


def test_decode_step_stores_then_attends(gpu_ops):
    lay = PageLayout(4, 128)
    gen = torch.Generator().manual_seed(613)
    cache = Cache(40, lay)
    table = random_tables(gen, [2500], 40)
    fill_sequence(gpu_ops, cache, gen, table[0], 2493)
    k = seeded_normal(gen, (7, 4, 128)).to(DEV)
    v = seeded_normal(gen, (7, 4, 128)).to(DEV)
    t = torch.arange(2493, 2500)
    slots = (table[0].long()[t // PAGE] * PAGE + t % PAGE).to(DEV)
    q = seeded_normal(gen, (7, 24, 128)).to(DEV)
    q8 = torch.empty((4, PAGE, 128), dtype=torch.int8, device=DEV)
    qs = torch.empty((4, PAGE), dtype=torch.float32, device=DEV)
    out = torch.full((7, 24, 128), float("nan"), dtype=torch.float16, device=DEV)
    gpu_ops.int8k_int4v_decode_step(q, k, v, slots, q8, qs, *cache.region_args(), table.to(DEV),
                                    torch.tensor([2500], dtype=torch.int32, device=DEV), None, None, None, None,
                                    None, out)
    blob = cache.blob()
    want_blob = blob.copy()
    geom = paged.Geometry(4, 128)
    paged.store(want_blob, geom, k.float().cpu().numpy(), v.float().cpu().numpy(), slots.cpu().numpy())
    assert np.array_equal(blob, want_blob), "decode_step store bytes"
    want = attention.decode_attention(q.float().cpu().numpy(), blob, geom, table.numpy(), [2500], 7)
    assert_close(out.float().cpu().numpy(), want, what="decode_step")


@pytest.mark.parametrize("hkv,d", [(4, 128), (2, 256)])
def test_k_and_v_halves_write_the_bytes_of_the_joint_store(gpu_ops, hkv, d):
    lay = PageLayout(hkv, d)
    gen = torch.Generator().manual_seed(614 + d)
    k = (torch.randn((300, hkv, d), generator=gen) * 2).to(torch.bfloat16).to(DEV)
    v = torch.randn((300, hkv, d), generator=gen).to(torch.bfloat16).to(DEV)
    slots = torch.randperm(16 * PAGE, generator=gen)[:300].to(torch.int64)
    slots[7] = -1
    slots[9] = 16 * PAGE + 5  # beyond the cache: skipped
    slots = slots.to(DEV)
    joint, halves = Cache(16, lay), Cache(16, lay)
    joint.store(gpu_ops, k, v, slots)
    h = halves.views
    gpu_ops.k_store_paged(k, slots, h["k"], h["k_scale"])
    gpu_ops.v_store_paged(v, slots, h["v"], h["v_scale"], h["v_zero"])
    assert np.array_equal(joint.blob(), halves.blob())
    only_k = Cache(16, lay)
    gpu_ops.k_store_paged(k, slots, only_k.views["k"], only_k.views["k_scale"])
    got = paged.regions(only_k.blob(), only_k.geom)
    assert not got["v"].any() and not got["v_scale"].any() and not got["v_zero"].any()
