"""Quantize-and-write kernel vs the oracle, byte for byte (GPU).

The cache is one byte allocation bound with ``bind_regions`` (the production
view), pre-filled with a marker byte so skipped writes are visible.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from k8v4_v030.cache_views import bind_regions
from k8v4_v030.layout import PAGE, PageLayout
from oracle import paged

pytestmark = pytest.mark.gpu

GOLD = json.loads((Path(__file__).parent / "golden" / "quant_known_answers.json").read_text())
DEV = "cuda"
MARK = 0xA5


def _cache(num_pages, layout):
    raw = torch.full((num_pages * layout.page_bytes,), MARK, dtype=torch.uint8, device=DEV)
    return raw, bind_regions(raw, layout)


def _store(ops, views, k, v, slots):
    ops.kv_store_paged(k, v, slots, views["k"], views["k_scale"], views["v"], views["v_scale"], views["v_zero"])


def _oracle_blob(num_pages, geom, k, v, slots):
    blob = paged.new_blob(num_pages, geom, fill=MARK)
    paged.store(blob, geom, k.float().cpu().numpy(), v.float().cpu().numpy(), slots.cpu().numpy())
    return blob


def _seeded_kv(seed, ntok, hkv, d, outliers=0.01, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(ntok, hkv, d, generator=g)
    v = torch.randn(ntok, hkv, d, generator=g)
    for t in (k, v):
        hit = torch.rand(t.shape, generator=g) < outliers
        t[hit] *= 20
    return k.to(dtype), v.to(dtype)


@pytest.mark.parametrize("hkv,d", [(4, 128), (2, 128), (4, 256), (2, 256)])
def test_store_bit_exact_random_slots(gpu_ops, hkv, d):
    layout = PageLayout(hkv, d)
    geom = paged.Geometry(hkv, d)
    num_pages, ntok = 40, 900
    print("store random hkv=%d d=%d" % (hkv, d), flush=True)
    k, v = _seeded_kv(1000 + hkv + d, ntok, hkv, d)
    g = torch.Generator().manual_seed(77)
    slots = torch.randperm(num_pages * 64, generator=g)[:ntok].to(torch.int64)
    slots[3] = -1
    slots[10] = -64
    slots[20] = num_pages * 64 + 5  # past the last page: skipped
    raw, views = _cache(num_pages, layout)
    _store(gpu_ops, views, k.to(DEV), v.to(DEV), slots.to(DEV))
    torch.cuda.synchronize()
    got = raw.cpu().numpy()
    want = _oracle_blob(num_pages, geom, k, v, slots)
    assert np.array_equal(got, want), "bytes differ at %s" % np.nonzero(got != want)[0][:10]


@pytest.mark.parametrize("d", [128, 256])
def test_store_known_answers(gpu_ops, d):
    layout = PageLayout(2, d)
    rows_k, rows_v = [], []
    for case in GOLD["k"]:
        rows_k.append(list(case["values"]) + [case.get("pad", 0.0)] * (d - len(case["values"])))
    for case in GOLD["v"]:
        rows_v.append(list(case["values"]) + [case.get("pad", 0.0)] * (d - len(case["values"])))
    n = max(len(rows_k), len(rows_v))
    rows_k += [[0.0] * d] * (n - len(rows_k))
    rows_v += [[0.0] * d] * (n - len(rows_v))
    # Token t, head 0 carries the case; head 1 repeats it negated.
    k = torch.tensor(rows_k, dtype=torch.float16)
    v = torch.tensor(rows_v, dtype=torch.float16)
    k = torch.stack([k, -k], dim=1)
    v = torch.stack([v, v], dim=1)
    slots = torch.arange(n, dtype=torch.int64)
    raw, views = _cache(1, layout)
    _store(gpu_ops, views, k.to(DEV), v.to(DEV), slots.to(DEV))
    torch.cuda.synchronize()
    for t, case in enumerate(GOLD["k"]):
        codes = views["k"][0, t, 0].cpu().tolist()
        assert codes[: len(case["codes"])] == case["codes"], case["name"]
        assert views["k"][0, t, 1].cpu().tolist()[: len(case["codes"])] == [-c for c in case["codes"]]
        assert float(views["k_scale"][0, t, 0]) == case["scale"], case["name"]
    for t, case in enumerate(GOLD["v"]):
        packed = views["v"][0, t, 0].cpu().numpy()
        nib = np.empty(d, dtype=np.uint8)
        nib[0::2], nib[1::2] = packed & 15, packed >> 4
        assert nib[: len(case["nibbles"])].tolist() == case["nibbles"], case["name"]
        assert float(views["v_scale"][0, t, 0]) == float(np.float32(case["scale"])), case["name"]
        assert float(views["v_zero"][0, t, 0]) == case["zero"], case["name"]


def test_store_bf16_and_strided_tokens(gpu_ops):
    layout = PageLayout(4, 128)
    geom = paged.Geometry(4, 128)
    ntok = 300
    k, v = _seeded_kv(5, ntok, 4, 128, dtype=torch.bfloat16)
    # K and V as slices of a wider fused projection (token stride != hkv*D).
    fused = torch.zeros(ntok, 24 * 128 + 2 * 512, dtype=torch.bfloat16)
    fused[:, 3072:3584] = k.reshape(ntok, 512)
    fused[:, 3584:4096] = v.reshape(ntok, 512)
    fused = fused.to(DEV)
    kd = fused[:, 3072:3584].view(ntok, 4, 128)
    vd = fused[:, 3584:4096].view(ntok, 4, 128)
    assert kd.stride(0) == 4096
    slots = torch.arange(ntok, dtype=torch.int64) * 3 % (8 * 64)
    raw, views = _cache(8, layout)
    _store(gpu_ops, views, kd, vd, slots.to(DEV))
    torch.cuda.synchronize()
    want = _oracle_blob(8, geom, k, v, slots)
    assert np.array_equal(raw.cpu().numpy(), want)


def test_store_rejects_bad_heads_and_dtypes(gpu_ops):
    layout = PageLayout(2, 128)
    raw, views = _cache(2, layout)
    slots = torch.arange(4, dtype=torch.int64, device=DEV)
    for hkv in (3, 8, 1):
        k = torch.randn(4, hkv, 128, dtype=torch.float16, device=DEV)
        with pytest.raises(RuntimeError, match=r"unsupported per-GPU KV head count %d \(this library serves 2 or 4\)" % hkv):
            _store(gpu_ops, views, k, k, slots)
    k = torch.randn(4, 2, 128, dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError):
        _store(gpu_ops, views, k, k, slots)
    k = torch.randn(4, 2, 128, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="int64"):
        _store(gpu_ops, views, k, k, slots.to(torch.int32))
    # Nothing was written by the refused calls.
    assert bool((raw == MARK).all())


def test_store_config2_full_size(gpu_ops):
    """4 sequences x 4,224 new tokens into a 16,384-page cache at random pages."""
    layout = PageLayout(4, 128)
    geom = paged.Geometry(4, 128)
    seqs, chunk, pool = 4, 4224, 16384
    print("store config2 full size", flush=True)
    k, v = _seeded_kv(1002, seqs * chunk, 4, 128)
    g = torch.Generator().manual_seed(1002)
    pages = torch.randperm(pool, generator=g)[: seqs * (chunk // 64)].view(seqs, chunk // 64)
    t = torch.arange(chunk)
    slots = torch.cat([pages[s, t // 64] * 64 + t % 64 for s in range(seqs)]).to(torch.int64)
    raw, views = _cache(pool, layout)
    _store(gpu_ops, views, k.to(DEV), v.to(DEV), slots.to(DEV))
    torch.cuda.synchronize()
    touched = torch.unique(slots // 64)
    page_bytes = layout.page_bytes
    got = raw.view(pool, page_bytes)[touched.to(DEV)].cpu().numpy()
    # Oracle on just the touched pages (renumbered), then compare page by page.
    remap = {int(p): i for i, p in enumerate(touched.tolist())}
    local = torch.tensor([remap[int(s) // 64] * 64 + int(s) % 64 for s in slots.tolist()], dtype=torch.int64)
    want = _oracle_blob(len(touched), geom, k, v, local).reshape(len(touched), page_bytes)
    assert np.array_equal(got, want)
    # Every other page is untouched.
    untouched_count = int((raw.view(pool, page_bytes) != MARK).any(dim=1).sum())
    assert untouched_count == len(touched)


def test_bound_store_matches_the_plain_op(gpu_ops):
    lay = PageLayout(4, 128)
    geom = paged.Geometry(4, 128)
    k, v = _seeded_kv(77, 300, 4, 128)
    slots = torch.randperm(20 * PAGE, generator=torch.Generator().manual_seed(78))[:300]
    a, va = _cache(20, lay)
    b, vb = _cache(20, lay)
    _store(gpu_ops, va, k.to(DEV), v.to(DEV), slots.to(DEV))
    call = gpu_ops.bind_kv_store_paged(k.to(DEV), v.to(DEV), slots.to(DEV), vb["k"], vb["k_scale"], vb["v"],
                                       vb["v_scale"], vb["v_zero"])
    call()
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert np.array_equal(b.view(torch.uint8).cpu().numpy(), _oracle_blob(20, geom, k, v, slots))
    assert gpu_ops.bind_kv_store_paged(k[:0].to(DEV), v[:0].to(DEV), slots[:0].to(DEV), vb["k"], vb["k_scale"],
                                       vb["v"], vb["v_scale"], vb["v_zero"]) is None


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_store_extreme_magnitudes_and_rounding_ties(gpu_ops, dtype):
    """Rows that stress every shortcut of the code evaluation, byte-compared with the oracle:
    tiny and huge magnitudes (bf16 subnormals, 1e37), constant rows, exact K ties
    (x = amax * (2k+1) / 254) and V values on rounding boundaries."""
    d, hkv = 128, 4
    layout = PageLayout(hkv, d)
    geom = paged.Geometry(hkv, d)
    g = torch.Generator().manual_seed(91)
    base = torch.randn(64, hkv, d, generator=g)
    rows_k, rows_v = [], []
    mags = [1e-40, 1e-38, 3e-5, 1.0, 300.0, 1e4] + ([1e20, 1e37] if dtype == torch.bfloat16 else [])
    for m in mags:
        rows_k.append(base[len(rows_k) % 64] * m)
        rows_v.append(base[(len(rows_v) + 7) % 64] * m)
    # exact half-way K codes: amax = 1, entries (2k+1)/254
    tie = torch.tensor([(2 * k + 1) / 254.0 for k in range(d)]).clamp(max=1.0)
    tie[0] = 1.0
    rows_k.append(tie.expand(hkv, d).clone())
    rows_v.append(torch.linspace(-1, 1, d).expand(hkv, d).clone())
    # constant rows and a V row whose values sit on code boundaries
    rows_k.append(torch.full((hkv, d), 0.25))
    rows_v.append(torch.full((hkv, d), -3.0))
    span = torch.arange(d, dtype=torch.float32) % 16 / 15.0 * 2 - 1
    rows_k.append(torch.zeros(hkv, d))
    rows_v.append((span + 1 / 30.0).expand(hkv, d).clone())
    k = torch.stack(rows_k).to(dtype)
    v = torch.stack(rows_v).to(dtype)
    n = k.shape[0]
    slots = torch.arange(n, dtype=torch.int64) * 5
    raw, views = _cache(4, layout)
    _store(gpu_ops, views, k.to(DEV), v.to(DEV), slots.to(DEV))
    torch.cuda.synchronize()
    want = _oracle_blob(4, geom, k, v, slots)
    got = raw.cpu().numpy()
    assert np.array_equal(got, want), "bytes differ at %s" % np.nonzero(got != want)[0][:10]
