"""Page geometry, slot addressing and MTP lengths (no GPU).

Constants come from tests/golden/reference_geometry.json, which restates the
numbers the reference's own tests pin (k8v4_v030/tests/test_layout_mtp.py).
The D=128 geometry is also checked against the oracle's independent byte math.
"""
from __future__ import annotations

import json
from pathlib import Path

import pytest

from k8v4_v030.layout import (
    CACHE_DTYPE,
    DECODE_MAX_T,
    GQA,
    HISTORIC_MTP_LEN,
    PAGE,
    SLOT_BYTES_PER_HEAD,
    PageLayout,
    as_int16,
    attention_pages_per_block,
    block_byte_span,
    builtin_q_end,
    element_byte,
    expand_block_ids,
    kernel_page_and_offset,
    max_kernel_pages,
    n_valid,
    page_regions,
    pages_per_block,
    region_stays_inside_block,
    region_view_specs,
    visible_lens,
)
from oracle import paged as opaged

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_geometry.json").read_text())
LAYOUTS = [PageLayout(h, d) for h in (2, 4) for d in (128, 256)]


def test_reference_d256_constants():
    assert GQA == 6 and SLOT_BYTES_PER_HEAD == GOLD["slot_bytes_per_head_d256"]
    for hkv in (2, 4):
        lay = PageLayout(hkv)
        want = GOLD["d256"]["hkv%d" % hkv]
        assert lay.head_dim == 256
        assert lay.hq == 6 * hkv
        assert lay.bytes_per_token == want["bytes_per_token"]
        assert lay.page_bytes == want["page_bytes"]
        assert lay.fp8_bytes_per_token == want["fp8_bytes_per_token"]
        assert lay.bytes_per_token < lay.fp8_bytes_per_token
    assert PageLayout(4).bytes_per_token > PageLayout(2).fp8_bytes_per_token
    assert CACHE_DTYPE == "int8_k_int4_v"


def test_d128_config_geometry_matches_oracle():
    want = GOLD["d128"]
    lay = PageLayout(4, 128)
    assert lay.slot_bytes_per_head == want["slot_bytes_per_head"]
    assert lay.bytes_per_token == want["hkv4"]["bytes_per_token"]
    assert lay.page_bytes == want["hkv4"]["page_bytes"]
    regions = page_regions(0, lay)
    for name, nbytes in want["hkv4"]["regions"].items():
        assert regions[name][1] == nbytes
    for lay in LAYOUTS:
        geom = opaged.Geometry(lay.hkv, lay.head_dim)
        assert geom.page_bytes == lay.page_bytes
        for name, off in geom.offsets().items():
            assert page_regions(3, lay)[name][0] == 3 * lay.page_bytes + off


def test_rejected_layouts():
    for bad in (1, 3, 8):
        with pytest.raises(ValueError):
            PageLayout(bad)
    with pytest.raises(ValueError):
        PageLayout(4, 64)
    with pytest.raises(ValueError):
        PageLayout.for_heads(12, 4)
    with pytest.raises(ValueError):
        PageLayout.for_heads(24, 2)
    assert PageLayout.for_heads(24, 4, 128) == PageLayout(4, 128)


def test_block_table_expansion_and_pages():
    for mb, kb, want in GOLD["attention_pages_per_block"]:
        assert attention_pages_per_block(mb, kb) == want
    for mml, mb, kb, want in GOLD["max_kernel_pages"]:
        assert max_kernel_pages(mml, mb, kb) == want
    for slot, page, off in GOLD["kernel_page_and_offset"]:
        assert kernel_page_and_offset(slot) == (page, off)
    for seq, page, want in GOLD["n_valid"]:
        assert n_valid(seq, page) == want
    e = GOLD["expand_block_ids"]
    assert expand_block_ids(e["ids"], e["ratio"]) == e["pages"]
    assert expand_block_ids([3, 5], 2)[1] == kernel_page_and_offset(3 * 128 + 70)[0]
    assert pages_per_block(64) == 1 and pages_per_block(1664) == 26
    with pytest.raises(ValueError):
        pages_per_block(100)
    with pytest.raises(ValueError):
        expand_block_ids([1], 0)


def test_region_specs_address_the_region_bytes():
    for lay in LAYOUTS:
        specs = region_view_specs(2, lay)
        assert element_byte(specs["k"], (1, 0, 0, 0)) == lay.page_bytes
        for name, (off, _len) in page_regions(0, lay).items():
            idx = (0, 0, 0, 0) if len(specs[name]["shape"]) == 4 else (0, 0, 0)
            assert element_byte(specs[name], idx) == off
        assert element_byte(specs["v_zero"], (0, 63, lay.hkv - 1)) == lay.page_bytes - 4
        # Every element of page 1 agrees with the oracle's longhand address math.
        geom = opaged.Geometry(lay.hkv, lay.head_dim)
        for tok in (0, 17, 63):
            for h in range(lay.hkv):
                assert element_byte(specs["k"], (1, tok, h, 5)) == opaged._byte_addr(geom, 1, tok, h, "k", 5)
                assert element_byte(specs["v"], (1, tok, h, 3)) == opaged._byte_addr(geom, 1, tok, h, "v", 3)
                for name in ("k_scale", "v_scale", "v_zero"):
                    assert element_byte(specs[name], (1, tok, h)) == opaged._byte_addr(geom, 1, tok, h, name)
        with pytest.raises(IndexError):
            element_byte(specs["k"], (2, 0, 0, 0))


def test_prefix_block_copy_keeps_pages_whole():
    for lay in LAYOUTS:
        for bs in (128, 1664, 2112):
            assert region_stays_inside_block(bs, lay)
        start, length = block_byte_span(2, 128, lay)
        assert (start, length) == (4 * lay.page_bytes, 2 * lay.page_bytes)


def test_mtp_visible_lens_are_full_width():
    vis = visible_lens(HISTORIC_MTP_LEN, 7)
    assert vis == GOLD["visible_lens_59500_q7"]
    assert as_int16(HISTORIC_MTP_LEN) == GOLD["as_int16_59500"]
    for j in range(7):
        assert vis[1 + j] == builtin_q_end(HISTORIC_MTP_LEN, 7, j)
        assert as_int16(vis[1 + j]) < 0 < vis[1 + j]
    assert visible_lens(70000, 7)[0] == 70000
    assert visible_lens(131072, 1) == [131072, 131072]
    assert visible_lens(3, 7)[1:4] == [1, 1, 1]
    assert DECODE_MAX_T == 10
    with pytest.raises(ValueError):
        visible_lens(100, 11)
    with pytest.raises(ValueError):
        visible_lens(100, 0)
    assert PAGE == 64
