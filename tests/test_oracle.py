"""Pins the CPU oracle before anything is compared against it (no GPU).

* quantization: hand-derived known answers (tests/golden/quant_known_answers.json),
  bit-identity of the vectorized and scalar restatements on random and
  tie-heavy rows, and round-trip error bounds;
* page bytes: the vectorized store equals the longhand byte packer;
* decode attention: reduction to torch's scaled_dot_product_attention on the
  dequantized tensors, closed forms (one visible key, identical keys),
  causality, MTP == serial q=1, explicit == builtin visible lengths, and
  agreement with the scalar ``causal_gqa`` restatement on tiny inputs;
* prefill attention: reduction to scaled_dot_product_attention with a
  bottom-right causal mask.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention, paged, quant, scalar

GOLD = json.loads((Path(__file__).parent / "golden" / "quant_known_answers.json").read_text())


def _row(case, d):
    vals = list(case["values"]) + [case.get("pad", 0.0)] * (d - len(case["values"]))
    return np.array(vals, dtype=np.float16).astype(np.float64)


@pytest.mark.parametrize("d", [128, 256])
def test_known_answer_k(d):
    for case in GOLD["k"]:
        row = _row(case, d)
        codes, scale = quant.quant_k(row[None])
        want = list(case["codes"]) + [0] * (d - len(case["codes"]))
        assert codes[0].tolist() == want, case["name"]
        assert float(scale[0]) == case["scale"], case["name"]
        s_codes, s_scale = scalar.quant_k(row.tolist())
        assert s_codes == want and s_scale == case["scale"]


@pytest.mark.parametrize("d", [128, 256])
def test_known_answer_v(d):
    for case in GOLD["v"]:
        row = _row(case, d)
        nib, scale, zero = quant.quant_v_nibbles(row[None])
        pad_code = case["nibbles"][0] if "pad" in case else None
        want = list(case["nibbles"])
        if pad_code is None:
            # zero padding: code of 0.0 under this row's scale/zero
            pad_code = int(min(15, max(0, math.floor(0.0 / case["scale"] + case["zero"] + 0.5))))
        want += [pad_code] * (d - len(want))
        assert nib[0].tolist() == want, case["name"]
        assert quant.stored_f32(scale)[0] == np.float32(case["scale"]), case["name"]
        assert float(zero[0]) == case["zero"], case["name"]
        packed, s_scale, s_zero = scalar.quant_v(row.tolist())
        assert packed == quant.pack_nibbles(nib)[0].tolist()
        assert s_zero == case["zero"]


def _adversarial_rows(rng, n, d):
    normal = rng.standard_normal((n, d)).astype(np.float16)
    out = normal.copy()
    out[rng.random((n, d)) < 0.01] *= 20
    ties = (rng.integers(-600, 600, (n, d)) / 256.0).astype(np.float16)  # many exact x.5 codes
    tiny = (rng.standard_normal((n, d)) * 1e-3).astype(np.float16)
    const = np.repeat(rng.standard_normal((n, 1)).astype(np.float16), d, axis=1)
    return np.concatenate([normal, out, ties, tiny, const]).astype(np.float64)


@pytest.mark.parametrize("d", [128, 256])
def test_vectorized_and_scalar_quant_are_bit_identical(d):
    rng = np.random.default_rng(1234 + d)
    rows = _adversarial_rows(rng, 24, d)
    kc, ks = quant.quant_k(rows)
    vp, vs, vz = quant.quant_v(rows)
    for i, row in enumerate(rows.tolist()):
        c, s = scalar.quant_k(row)
        assert kc[i].tolist() == c and ks[i] == s
        p, s2, z2 = scalar.quant_v(row)
        assert vp[i].tolist() == p and vs[i] == s2 and vz[i] == z2


def test_roundtrip_error_bounds():
    rng = np.random.default_rng(7)
    rows = _adversarial_rows(rng, 32, 128)[:-32]  # constant rows have their own known answers
    kc, ks = quant.quant_k(rows)
    err = np.abs(rows - quant.dequant_k(kc, ks))
    assert np.all(err <= 0.5 * ks[:, None] * (1 + 1e-9) + 1e-300)
    vp, vs, vz = quant.quant_v(rows)
    verr = np.abs(rows - quant.dequant_v(vp, vs, vz))
    assert np.all(verr <= 0.5 * vs[:, None] * (1 + 1e-9) + 1e-12)
    assert np.all(quant.unpack_nibbles(vp) <= 15)


@pytest.mark.parametrize("hkv,d", [(2, 256), (4, 128)])
def test_vectorized_store_equals_byte_packer(hkv, d):
    geom = paged.Geometry(hkv, d)
    rng = np.random.default_rng(3)
    n = 150
    k = rng.standard_normal((n, hkv, d)).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    slots = rng.permutation(4 * 64)[:n].astype(np.int64)
    slots[5] = -1
    slots[9] = 4 * 64 + 3  # past the last page: skipped
    a = paged.new_blob(4, geom, fill=0xAB)
    b = paged.new_blob(4, geom, fill=0xAB)
    paged.store(a, geom, k, v, slots)
    for t in range(n):
        if slots[t] < 4 * 64:
            paged.write_token(b, geom, int(slots[t]), k[t].astype(np.float64), v[t].astype(np.float64))
    assert np.array_equal(a, b)
    keys, vals = paged.read_token(a, geom, int(slots[0]))
    ks = quant.quant_k(k[0].astype(np.float64))[1]
    for h in range(hkv):
        assert np.max(np.abs(keys[h] - k[0, h])) <= ks[h] * 0.5 + 1e-6
    untouched = paged.new_blob(4, geom, fill=0xAB)
    paged.store(untouched, geom, k[:1], v[:1], np.array([-3]))
    assert np.all(untouched == 0xAB)


def _random_cache(geom, seq_lens, rng, pool_extra=3, ppb=1):
    """Store N(0,1) fp16 K/V for each sequence at random distinct pages."""
    pages = [(L + 63) // 64 for L in seq_lens]
    width = max(1, max(-(-p // ppb) for p in pages))
    n_blocks = sum(-(-p // ppb) for p in pages) + pool_extra
    perm = rng.permutation(n_blocks)
    table = np.zeros((len(seq_lens), width), dtype=np.int32)
    blob = paged.new_blob(n_blocks * ppb, geom)
    cur = 0
    kv = []
    for b, L in enumerate(seq_lens):
        nb = -(-pages[b] // ppb)
        table[b, :nb] = perm[cur : cur + nb]
        cur += nb
        k = rng.standard_normal((L, geom.hkv, geom.d)).astype(np.float16)
        v = rng.standard_normal((L, geom.hkv, geom.d)).astype(np.float16)
        t = np.arange(L)
        slots = (table[b, (t // 64) // ppb].astype(np.int64) * ppb + (t // 64) % ppb) * 64 + t % 64
        paged.store(blob, geom, k, v, slots)
        kv.append((k, v))
    return blob, table, kv


def _sdpa_reference(q_deq, k, v, ends):
    """torch SDPA (float64, CPU) with per-row key ends; GQA by repeat_interleave."""
    hq = q_deq.shape[1]
    hkv = k.shape[1]
    qt = torch.from_numpy(q_deq).permute(1, 0, 2)[None]  # [1, HQ, R, D]
    kt = torch.from_numpy(k).repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2)[None]
    vt = torch.from_numpy(v).repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2)[None]
    S = k.shape[0]
    allow = torch.arange(S)[None, :] < torch.as_tensor(ends)[:, None]
    mask = torch.zeros(allow.shape, dtype=torch.float64).masked_fill(~allow, float("-inf"))
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=1.0 / math.sqrt(k.shape[2]))
    return out[0].permute(1, 0, 2).numpy()


@pytest.mark.parametrize("hkv,d,q_len", [(4, 128, 7), (2, 256, 1), (4, 128, 3)])
def test_decode_equals_sdpa_on_dequantized_tensors(hkv, d, q_len):
    geom = paged.Geometry(hkv, d)
    rng = np.random.default_rng(11 + q_len)
    seq_lens = [70, 200]
    blob, table, _ = _random_cache(geom, seq_lens, rng)
    q = rng.standard_normal((len(seq_lens) * q_len, 6 * hkv, d)).astype(np.float16)
    got = attention.decode_attention(q, blob, geom, table, seq_lens, q_len)
    for b, L in enumerate(seq_lens):
        k, v = paged.gather_dequant(blob, geom, table[b], L, 1)
        rows = q[b * q_len : (b + 1) * q_len].astype(np.float64)
        qc, qs = quant.quant_k(rows)
        q_deq = qc.astype(np.float64) * qs[..., None]
        k64 = paged.gather_codes(blob, geom, table[b], 0, L, 1)
        kd = k64[0].astype(np.float64) * k64[1].astype(np.float64)[..., None]
        ends = [L - q_len + j + 1 for j in range(q_len)]
        want = _sdpa_reference(q_deq, kd, v.astype(np.float64), ends)
        np.testing.assert_allclose(got[b * q_len : (b + 1) * q_len], want, atol=1e-12, rtol=1e-9)


def test_decode_closed_forms_and_masking():
    geom = paged.Geometry(2, 128)
    rng = np.random.default_rng(5)
    blob, table, _ = _random_cache(geom, [130], rng)
    q = rng.standard_normal((7, 12, 128)).astype(np.float16)
    # One visible key: the output is that key's dequantized value row.
    vis = np.array([[1] * 8], dtype=np.int64)
    out = attention.decode_attention(q, blob, geom, table, [130], 7, visible=vis)
    _, v = paged.gather_dequant(blob, geom, table[0], 1, 1)
    for h in range(12):
        np.testing.assert_allclose(out[:, h], np.repeat(v[0:1, h // 6], 7, 0), rtol=0, atol=1e-7)
    # Zero visible keys -> zeros.
    out0 = attention.decode_attention(q, blob, geom, table, [130], 7, visible=np.zeros((1, 8), np.int64))
    assert np.all(out0 == 0)
    # Explicit visible lengths equal to the builtin ones give the same output.
    L = 130
    builtin = attention.decode_attention(q, blob, geom, table, [L], 7)
    ends = [max(1, L - (6 - j)) for j in range(7)]
    explicit = attention.decode_attention(q, blob, geom, table, [L], 7, visible=np.array([[max(ends)] + ends]))
    np.testing.assert_array_equal(builtin, explicit)
    # MTP-7 equals seven q=1 calls with shortened lengths.
    for j in range(7):
        one = attention.decode_attention(q[j : j + 1], blob, geom, table, [L - 6 + j], 1)
        np.testing.assert_allclose(builtin[j], one[0], atol=1e-12)


def test_identical_keys_average_values():
    geom = paged.Geometry(2, 128)
    blob = paged.new_blob(2, geom)
    rng = np.random.default_rng(9)
    krow = rng.standard_normal((1, 2, 128)).astype(np.float16)
    vals = rng.standard_normal((40, 2, 128)).astype(np.float16)
    paged.store(blob, geom, np.repeat(krow, 40, 0), vals, np.arange(40))
    q = rng.standard_normal((1, 12, 128)).astype(np.float16)
    out = attention.decode_attention(q, blob, geom, np.array([[0, 1]]), [40], 1)
    _, v = paged.gather_dequant(blob, geom, np.array([0, 1]), 40, 1)
    for h in range(12):
        np.testing.assert_allclose(out[0, h], v[:, h // 6].astype(np.float64).mean(0), atol=1e-9)


def test_oracle_agrees_with_scalar_causal_gqa_and_causality():
    geom = paged.Geometry(2, 128)
    key = np.array(scalar.deterministic_rows(5, 2, seed=1, dim=128))
    value = np.array(scalar.deterministic_rows(5, 2, seed=2, dim=128))
    q_rows = np.repeat(key[3:5], 6, axis=1)  # [2, 12, 128]: query = the last two keys per head
    want = np.array(scalar.causal_gqa(q_rows.tolist(), key.tolist(), value.tolist(), 5, 2))
    blob = paged.new_blob(1, geom)
    paged.store(blob, geom, key, value, np.arange(5))
    got = attention.decode_attention(q_rows, blob, geom, np.array([[0]]), [5], 2)
    # The scalar restatement keeps double scales; the oracle reads the stored fp32 planes.
    np.testing.assert_allclose(got, want, atol=2e-6)
    key_cut = key.copy()
    key_cut[-1] = 0.0
    cut = np.array(scalar.causal_gqa(q_rows.tolist(), key_cut.tolist(), value.tolist(), 5, 2))
    assert np.array_equal(cut[0], want[0])
    assert not np.array_equal(cut[1], want[1])


def test_prefill_equals_sdpa_bottom_right():
    geom = paged.Geometry(4, 128)
    rng = np.random.default_rng(21)
    L, q_len, ppb = 150, 40, 2
    blob, table, _ = _random_cache(geom, [L], rng, ppb=ppb)
    q = rng.standard_normal((q_len, 24, 128)).astype(np.float16)
    got = attention.prefill_attention(q, blob, geom, table[0], L, ppb, 1 / math.sqrt(128))
    k, v = paged.gather_dequant(blob, geom, table[0], L, ppb)
    ends = [L - q_len + r + 1 for r in range(q_len)]
    want = _sdpa_reference(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), ends)
    np.testing.assert_allclose(got, want, atol=1e-12, rtol=1e-9)
    rows = np.array([0, 17, 39])
    sub = attention.prefill_attention(q, blob, geom, table[0], L, ppb, 1 / math.sqrt(128), rows=rows)
    np.testing.assert_allclose(sub, got[rows], atol=1e-12)


# ---------------------------------------------------------------- torch CPU baseline
def test_torch_cpu_store_writes_the_oracle_bytes():
    """The CPU baseline's vectorized store (bench.py's cpu_baseline) is bit-exact
    to the oracle's, including exact ties, constant rows, skipped slots and bf16 input."""
    import torch

    from oracle import torch_cpu

    geom = paged.Geometry(4, 128)
    rng = np.random.default_rng(33)
    key = (rng.standard_normal((90, 4, 128)) * 3).astype(np.float16)
    value = rng.standard_normal((90, 4, 128)).astype(np.float16)
    key[5, 1, :4] = [127.0, 0.5, 1.5, -0.5]
    key[5, 1, 4:] = 0
    value[6, 2] = 1.25  # constant row: scale floor 1e-8
    key[7] = 0  # zero rows: codes 0, scale 0
    slots = rng.permutation(4 * 64)[:90].astype(np.int64)
    slots[3], slots[4] = -1, 4 * 64 + 9
    want = paged.new_blob(4, geom)
    paged.store(want, geom, key, value, slots)
    raw = torch.zeros(4 * geom.page_bytes, dtype=torch.uint8)
    torch_cpu.store(torch_cpu.region_views(raw, geom), torch.from_numpy(key), torch.from_numpy(value),
                    torch.from_numpy(slots))
    assert np.array_equal(raw.numpy(), want)
    bf = torch.from_numpy(key.astype(np.float32)).to(torch.bfloat16)
    want_bf = paged.new_blob(4, geom)
    paged.store(want_bf, geom, bf.float().numpy(), value, slots)
    raw.zero_()
    torch_cpu.store(torch_cpu.region_views(raw, geom), bf, torch.from_numpy(value), torch.from_numpy(slots))
    assert np.array_equal(raw.numpy(), want_bf)


def test_torch_cpu_decode_and_prefill_match_the_oracle():
    """fp32 torch decode (int8 Q) and key-tiled prefill agree with the float64
    oracle; a 64-token key tile makes the prefill cross many tiles and row groups."""
    import torch

    from oracle import torch_cpu

    geom = paged.Geometry(2, 256)
    rng = np.random.default_rng(34)
    lengths = [700, 65, 0, 300]
    blob, table, _ = _random_cache(geom, lengths, rng, ppb=2)
    views = torch_cpu.region_views(torch.from_numpy(blob.copy()), geom)
    q = rng.standard_normal((4 * 7, 12, 256)).astype(np.float16)
    want = attention.decode_attention(q, blob, geom, table, lengths, 7, 2)
    got = torch_cpu.decode(views, torch.from_numpy(q), torch.from_numpy(table), lengths, 7, 2)
    np.testing.assert_allclose(got.numpy(), want, atol=2e-5, rtol=1e-4)
    qp = rng.standard_normal((300, 12, 256)).astype(np.float16)
    scale = 1 / math.sqrt(256)
    want_p = attention.prefill_attention(qp, blob, geom, table[0], 700, 2, scale)
    old = torch_cpu.KEY_TILE, torch_cpu.ROW_GROUP
    try:
        torch_cpu.KEY_TILE, torch_cpu.ROW_GROUP = 64, 96
        got_p = torch_cpu.prefill(views, torch.from_numpy(qp), torch.from_numpy(table[0]), 700, scale, 2)
    finally:
        torch_cpu.KEY_TILE, torch_cpu.ROW_GROUP = old
    np.testing.assert_allclose(got_p.numpy(), want_p, atol=2e-5, rtol=1e-4)
