"""The C ABI library without a GPU: it loads, exports every declared symbol with
the argument count ops_api binds, and its host-side argument checks reject bad
calls with the reference's messages before any device work is enqueued."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from k8v4_v030 import ops_api

HEADER = Path(__file__).resolve().parents[1] / "include" / "k8v4_abi.h"


def _declared() -> dict[str, int]:
    """Function name -> parameter count, parsed from the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(k8v4_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    path = Path(ops_api.library_path())
    if not path.is_file():
        pytest.skip("library not built (run __graft_entry__.build())")
    return ops_api.load_library()


def test_header_declares_the_entry_points():
    names = set(_declared())
    assert {"k8v4_abi_version", "k8v4_last_error", "k8v4_kv_store_paged", "k8v4_attn_batch",
            "k8v4_attn_batch_profiled", "k8v4_attn_workspace_bytes", "k8v4_prefill_paged",
            "k8v4_prefill_workspace_bytes"} <= names


def test_every_declared_symbol_is_exported_and_bound(lib):
    bound = {"k8v4_kv_store_paged": lib.k8v4_kv_store_paged.argtypes}
    for name, argtypes, _ in ops_api._EXTRA_SYMBOLS:
        bound[name] = argtypes
    for name, nparams in _declared().items():
        fn = getattr(lib, name)  # AttributeError if not exported
        assert fn is not None
        if name in bound:
            assert len(bound[name]) == nparams, name
    assert lib.k8v4_abi_version() == 3


def _attn(lib, **over):
    """k8v4_attn_batch with plausible host arguments and fake (never dereferenced) pointers."""
    p = 0x10000
    a = dict(q=p, q_dtype=0, q_tok_stride=24 * 128, k_cache=p, k_scale=p, v_cache=p, v_scale=p,
             v_zero=p, num_pages=64, ks=52224, kss=52224, vs=52224, vss=52224, vzs=52224, bt=p,
             bt_stride=32, width=32, ppb=1, seq=p, vis=None, vis_stride=0, batch=1, q_len=1, hkv=4,
             d=128, out=p, out_dtype=0, out_stride=24 * 128, ws=p, ws_bytes=0, splits=0, stream=None)
    a.update(over)
    return lib.k8v4_attn_batch(*a.values())


@pytest.mark.parametrize("hkv", [1, 3, 8])
def test_attn_rejects_head_counts_with_the_reference_message(lib, hkv):
    assert _attn(lib, hkv=hkv) == 1
    msg = lib.k8v4_last_error().decode()
    assert msg == "unsupported per-GPU KV head count %d (this library serves 2 or 4)" % hkv


def test_attn_host_checks(lib):
    assert _attn(lib, q_len=11) == 1 and "q_len*GQA exceeds BM" in lib.k8v4_last_error().decode()
    assert _attn(lib, d=64) == 1 and "head dim" in lib.k8v4_last_error().decode()
    assert _attn(lib, q=0x10008) == 1 and "16-byte" in lib.k8v4_last_error().decode()
    assert _attn(lib, bt_stride=8) == 1 and "block_table" in lib.k8v4_last_error().decode()
    assert _attn(lib, q_dtype=2) == 1 and "q dtype" in lib.k8v4_last_error().decode()
    assert _attn(lib, ws=0) == 1 and "null" in lib.k8v4_last_error().decode()


def test_store_rejects_head_counts(lib):
    p = 0x10000
    rc = lib.k8v4_kv_store_paged(p, p, 0, 3 * 128, 3 * 128, p, 10, 3, 128, p, p, p, p, p, 64,
                                 52224, 52224, 52224, 52224, 52224, None)
    assert rc == 1
    assert "unsupported per-GPU KV head count 3" in lib.k8v4_last_error().decode()


def test_workspace_bytes_rejects_bad_shapes(lib):
    assert lib.k8v4_attn_workspace_bytes(0, 32, 1, 1, 4, 128, 0) == -1
    assert lib.k8v4_attn_workspace_bytes(1, 32, 1, 1, 3, 128, 0) == -1
    assert lib.k8v4_attn_workspace_bytes(1, 32, 1, 1, 4, 96, 0) == -1
    # An explicit split count fixes the size: splits x hkv x q_len x 6 x (2 D + 8) bytes.
    assert lib.k8v4_attn_workspace_bytes(4, 2048, 1, 7, 4, 128, 64) == 64 * 4 * 7 * 6 * (2 * 128 + 8)


@pytest.mark.parametrize("hkv,d,q_len,splits", [(4, 128, 7, 64), (2, 256, 7, 512), (4, 128, 1, 3),
                                                 (2, 128, 10, 17), (4, 256, 4, 256)])
def test_workspace_bytes_match_the_python_sizing(lib, hkv, d, q_len, splits):
    """The host-side sizing (plan.attn_workspace_bytes, used by the backend's
    scratch) and the library agree for an explicit split count."""
    from k8v4_v030.layout import PageLayout
    from k8v4_v030.plan import attn_workspace_bytes, query_tile_bytes, split_state_bytes

    lay = PageLayout(hkv, d)
    got = lib.k8v4_attn_workspace_bytes(1, 4096, 1, q_len, hkv, d, splits)
    head = query_tile_bytes(1, lay)
    assert got == attn_workspace_bytes(splits, q_len, lay) == head + splits * split_state_bytes(q_len, lay)
    # Only the paired-halves shapes (head dim 256) quantize their query into
    # the workspace: 64 rows of 256 codes and 64 scales per head.
    assert head == (hkv * (64 * 256 + 256) if d == 256 else 0)
    assert split_state_bytes(q_len, lay) % 16 == 0  # every split state starts 16-byte aligned
    # The grid never has fewer splits than sequences.
    assert lib.k8v4_attn_workspace_bytes(8, 4096, 1, q_len, hkv, d, 3) == attn_workspace_bytes(8, q_len, lay, 8)


def test_ops_layer_raises_without_gpu_tensors(lib):
    import torch

    from k8v4_v030.cache_views import bind_regions
    from k8v4_v030.layout import PageLayout

    lay = PageLayout(4, 128)
    v = bind_regions(torch.zeros(2 * lay.page_bytes, dtype=torch.int8), lay)
    k = torch.zeros(3, 4, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        ops_api.ops().kv_store_paged(k, k, torch.zeros(3, dtype=torch.int64), v["k"], v["k_scale"], v["v"],
                                     v["v_scale"], v["v_zero"])


def test_q_quant_host_checks(lib):
    p = 0x10000
    assert lib.k8v4_q_quant(p, 0, 0, 24 * 128, 7, 3, 128, p, p, None) == 1
    assert "unsupported per-GPU KV head count 3" in lib.k8v4_last_error().decode()
    assert lib.k8v4_q_quant(p, 0, 0, 24 * 128, 11, 4, 128, p, p, None) == 1
    assert lib.k8v4_last_error().decode() == "tq*GQA exceeds BM"
    assert lib.k8v4_q_quant(p, 0, 5, 0, 0, 4, 128, p, p, None) == 1
    assert "unknown query layout" in lib.k8v4_last_error().decode()
    assert lib.k8v4_q_quant(p, 2, 1, 0, 0, 4, 128, p, p, None) == 1
    assert "q dtype" in lib.k8v4_last_error().decode()


def test_attn_q8_host_checks(lib):
    p = 0x10000
    args = [p, p, 4 * 64 * 128, 4 * 64, p, p, p, p, p, 64, 52224, 52224, 52224, 52224, 52224, p, 32, 32, 1, p,
            None, 0, 1, 7, 4, 128, p, 0, 24 * 128, p, 1 << 20, 0, None]
    bad = list(args)
    bad[0] = None
    assert lib.k8v4_attn_batch_q8(*bad) == 1 and "null" in lib.k8v4_last_error().decode()
    bad = list(args)
    bad[2] = 64 * 128  # one head's tile per sequence: too short
    assert lib.k8v4_attn_batch_q8(*bad) == 1 and "q8 must be" in lib.k8v4_last_error().decode()
    bad = list(args)
    bad[24] = 3
    assert lib.k8v4_attn_batch_q8(*bad) == 1
    assert "unsupported per-GPU KV head count 3" in lib.k8v4_last_error().decode()


def test_unpaged_stage_ops_raise_with_a_pointer_to_the_paged_ones(lib):
    o = ops_api.ops()
    for name, hint in (("k_store", "k_store_paged"), ("v_store", "v_store_paged"),
                       ("int8k_int4v_s1", "int8k_int4v_s1_paged")):
        with pytest.raises(RuntimeError, match="%s: the reference's unpaged single-page op.*use %s" % (name, hint)):
            getattr(o, name)(None, None, None)


def test_every_reference_op_name_is_in_the_table(lib):
    """The schema list of torch.ops.xe2_kv (xe2_kv_ops.cpp:1779-1822)."""
    names = ["q_quant_once", "k_store", "v_store", "int8k_int4v_s1", "k_store_paged", "v_store_paged",
             "kv_store_paged", "int8k_int4v_s1_paged", "int8k_int4v_s1_varlen_paged",
             "int8k_int4v_s1_varlen_from_q", "int8k_int4v_decode_step", "int8k_int4v_attn_batch"]
    o = ops_api.ops()
    assert all(callable(getattr(o, n)) for n in names)


def _prefill_batch(lib, tok0, q_lens, seq_lens, rows, **over):
    """k8v4_prefill_paged_batch with plausible host arguments and fake (never dereferenced) pointers."""
    import ctypes

    p = 0x10000
    n = len(tok0)
    arrs = [(ctypes.c_int64 * max(n, 1))(*v) for v in (tok0, q_lens, seq_lens, rows)]
    a = dict(q=p, q_dtype=0, q_tok_stride=24 * 128, k_cache=p, k_scale=p, v_cache=p, v_scale=p, v_zero=p,
             num_pages=64, ks=52224, kss=52224, vs=52224, vss=52224, vzs=52224, bt=p, bt_stride=32, width=32,
             ppb=1, nseq=n, tok0=ctypes.cast(arrs[0], ctypes.c_void_p), q_lens=ctypes.cast(arrs[1], ctypes.c_void_p),
             seq_lens=ctypes.cast(arrs[2], ctypes.c_void_p), rows=ctypes.cast(arrs[3], ctypes.c_void_p), hkv=4,
             d=128, scale=0.088, out=p, out_dtype=0, out_stride=24 * 128, ws=p, ws_bytes=0, stream=None)
    a.update(over)
    return lib.k8v4_prefill_paged_batch(*a.values())


def test_prefill_batch_host_checks(lib):
    """The batched prefill checks each sequence like the single entry, before any launch."""
    assert _prefill_batch(lib, [], [], [], []) == 0  # nothing to do
    assert _prefill_batch(lib, [0], [5], [100], [0], hkv=3) == 1
    assert "unsupported per-GPU KV head count 3" in lib.k8v4_last_error().decode()
    assert _prefill_batch(lib, [0, 9], [5, 9], [100, 8], [0, 1]) == 1
    assert "sequence 1: query longer than the KV sequence" in lib.k8v4_last_error().decode()
    assert _prefill_batch(lib, [0], [5], [64 * 32 + 1], [0]) == 1
    assert "block table row covers 2048 tokens" in lib.k8v4_last_error().decode()
    assert _prefill_batch(lib, [0], [5], [100], [-1]) == 1
    assert "negative" in lib.k8v4_last_error().decode()
    assert _prefill_batch(lib, [0], [5], [100], [0], bt_stride=16) == 1
    assert "stride" in lib.k8v4_last_error().decode()
    assert _prefill_batch(lib, [0], [5], [100], [0], q=0x10008) == 1
    assert "16-byte" in lib.k8v4_last_error().decode()
    # A workspace smaller than one launch's partial states: K8V4_ERR_WORKSPACE, nothing launched.
    assert _prefill_batch(lib, [0], [5], [100], [0], ws_bytes=1024) == 2
    assert "prefill workspace holds 1024 bytes" in lib.k8v4_last_error().decode()
    # Eleven sequences are two launches; the second's sequence is too large for
    # the schedule.  Every launch is planned before the first is enqueued, so
    # the call fails on the plan (on a host without a GPU an enqueued launch
    # would have failed first, with a launch error).
    n, big = 11, (1 << 30) - 1
    assert _prefill_batch(lib, [0] * n, [5] * (n - 1) + [1 << 20], [100] * (n - 1) + [big], list(range(n)),
                          ppb=1 << 20, ws_bytes=1 << 30) == 1
    assert "sequence 10 too large for one call" in lib.k8v4_last_error().decode()


def test_prefill_batch_workspace_covers_every_short_single_call(lib):
    for hkv, d in ((4, 128), (2, 128), (2, 256), (4, 256)):
        need = lib.k8v4_prefill_batch_workspace_bytes(hkv, d)
        assert need > 0
        for q_len, seq_len in ((1, 64), (40, 2000), (128, 9000)):  # up to three row blocks: no tile pre-pass
            assert lib.k8v4_prefill_workspace_bytes(seq_len, q_len, hkv, d) <= need
    assert lib.k8v4_prefill_batch_workspace_bytes(3, 128) == -1
    assert lib.k8v4_prefill_batch_workspace_bytes(4, 64) == -1


@pytest.mark.parametrize("hkv,d,q_len,ctx,tiles", [
    # head dim 128: tile images from four 256-row blocks on (q_len > 128)
    (4, 128, 128, 4096, False), (4, 128, 129, 4096, True), (2, 128, 4224, 131072, True),
    # head dim 256: only where the per-head pre-pass pays for itself
    (2, 256, 128, 4096, False), (2, 256, 512, 4096, False), (2, 256, 512, 16384, False),
    (2, 256, 512, 65536, True), (2, 256, 2048, 16384, True), (2, 256, 4224, 131072, True),
    (4, 256, 128, 65536, False), (4, 256, 4224, 65536, True),
])
def test_single_prefill_uses_tile_images_where_they_pay(lib, hkv, d, q_len, ctx, tiles):
    """The single prefill entry's plan (the library's): pages dequantized once
    per KV head into tile images beside the partial states, or converted in
    place like the batched entry (the backend sends only the latter to one
    batched launch)."""
    seq_len = ctx + q_len
    assert lib.k8v4_prefill_uses_tiles(seq_len, q_len, hkv, d) == int(tiles)
    if tiles:  # the workspace holds one tile image per page beside the partial states
        stride = 35 * 1024 if d == 128 else 68 * 1024
        assert lib.k8v4_prefill_workspace_bytes(seq_len, q_len, hkv, d) > -(-seq_len // 64) * stride
    assert lib.k8v4_prefill_uses_tiles(seq_len, seq_len + 1, hkv, d) == -1
