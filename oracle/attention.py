"""Attention over the quantized paged cache, computed in float64 on the CPU.

Decode / MTP verify (reference: k8v4_v030/oracle.py:100-163 for the math,
native/xe2_kv_ops.cpp:657-791 and :1081-1166 for the batch semantics):

* every query row (token j, query head h) is quantized with the K rule
  (``quant.quant_k``) -- int8 codes and a double scale;
* query head h reads KV head h // 6;
* score(t) = (exact integer dot of the codes) * q_scale * k_scale[t] / sqrt(D),
  with k_scale the stored fp32;
* key t is visible to token j iff ``t < L0`` and ``t < end_j``, where
  ``L0 = visible[b][0]`` and ``end_j = visible[b][1 + j]`` when ``visible`` is
  given, else ``L0 = seq_len`` and ``end_j = seq_len - q_len + j + 1``;
* softmax in float64; a row with no visible key returns zeros;
* V is dequantized in fp32 from the stored codes and planes (dequant.py:96-106).

Chunked prefill (reference: dequant.py:245-261, :448-501 and
onednn_prefill.py:89-121): fp query (no quantization), fp32-dequantized K/V,
query row r of a q_len suffix sees keys ``t <= seq_len - q_len + r``.
"""
from __future__ import annotations

import numpy as np

from . import paged, quant

GQA = 6


def _softmax_rows(scores: np.ndarray) -> np.ndarray:
    """Row softmax with -inf masking; all-masked rows give zeros."""
    top = np.max(scores, axis=-1, keepdims=True)
    dead = ~np.isfinite(top)
    top = np.where(dead, 0.0, top)
    e = np.exp(scores - top)
    total = e.sum(axis=-1, keepdims=True)
    return np.where(total > 0.0, e / np.where(total > 0.0, total, 1.0), 0.0)


def decode_attention(
    q,
    blob: np.ndarray,
    geom: paged.Geometry,
    block_table,
    seq_lens,
    q_len: int,
    pages_per_block: int = 1,
    visible=None,
) -> np.ndarray:
    """``q[B*q_len, HQ, D]`` -> float64 output of the same shape."""
    q = np.asarray(q, dtype=np.float64)
    block_table = np.asarray(block_table)
    seq_lens = np.asarray(seq_lens, dtype=np.int64).reshape(-1)
    b_count = block_table.shape[0]
    hq, d = q.shape[1], q.shape[2]
    if hq != GQA * geom.hkv or d != geom.d:
        raise ValueError("query heads/dim do not match the geometry")
    if q.shape[0] != b_count * q_len:
        raise ValueError("query rows must be batch * q_len")
    out = np.zeros(q.shape, dtype=np.float64)
    inv_sqrt = 1.0 / np.sqrt(float(d))
    table_pages = block_table.shape[1] * int(pages_per_block)
    for b in range(b_count):
        if visible is not None:
            vis = np.asarray(visible[b], dtype=np.int64)
            l0 = int(vis[0])
            ends = [int(vis[1 + j]) for j in range(q_len)]
        else:
            l0 = int(seq_lens[b])
            ends = [l0 - q_len + j + 1 for j in range(q_len)]
        n = max(0, min(l0, table_pages * paged.PAGE))
        if n == 0:
            continue
        k8, ks, vn, vs, vz = paged.gather_codes(blob, geom, block_table[b], 0, n, pages_per_block)
        _, v = paged.dequant_f32(k8, ks, vn, vs, vz)
        v = v.astype(np.float64)
        kf = k8.astype(np.float64)
        ksd = ks.astype(np.float64)
        rows = q[b * q_len : (b + 1) * q_len]  # [q_len, HQ, D]
        qc, qs = quant.quant_k(rows)  # codes [q_len, HQ, D], scale [q_len, HQ]
        t = np.arange(n)
        for g in range(geom.hkv):
            heads = slice(g * GQA, (g + 1) * GQA)
            qg = qc[:, heads].astype(np.float64).reshape(q_len * GQA, d)
            dots = (qg @ kf[:, g].T).reshape(q_len, GQA, n)  # exact: |dot| < 2^22
            scores = dots * qs[:, heads, None] * ksd[None, None, :, g] * inv_sqrt
            limit = np.minimum(np.asarray(ends)[:, None], n)  # [q_len, 1]
            scores = np.where((t[None, :] < limit)[:, None, :], scores, -np.inf)
            p = _softmax_rows(scores)
            out[b * q_len : (b + 1) * q_len, heads] = p @ v[:, g]
    return out


def prefill_attention(
    q,
    blob: np.ndarray,
    geom: paged.Geometry,
    block_row,
    seq_len: int,
    pages_per_block: int,
    scale: float,
    rows=None,
) -> np.ndarray:
    """``q[q_len, HQ, D]`` (the last q_len tokens) -> float64 ``[len(rows), HQ, D]``."""
    q = np.asarray(q, dtype=np.float64)
    q_len, hq, d = q.shape
    if hq != GQA * geom.hkv or d != geom.d:
        raise ValueError("query heads/dim do not match the geometry")
    if q_len > seq_len:
        raise ValueError("query longer than the KV sequence")
    rows = np.arange(q_len) if rows is None else np.asarray(rows, dtype=np.int64)
    k, v = paged.gather_dequant(blob, geom, block_row, seq_len, pages_per_block)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    t = np.arange(seq_len)
    allow = t[None, :] <= (seq_len - q_len + rows)[:, None]  # [R, S]
    out = np.zeros((rows.size, hq, d), dtype=np.float64)
    for g in range(geom.hkv):
        heads = slice(g * GQA, (g + 1) * GQA)
        qg = q[rows][:, heads]  # [R, 6, D]
        scores = (qg.reshape(-1, d) @ k[:, g].T).reshape(rows.size, GQA, seq_len) * float(scale)
        scores = np.where(allow[:, None, :], scores, -np.inf)
        out[:, heads] = _softmax_rows(scores) @ v[:, g]
    return out
