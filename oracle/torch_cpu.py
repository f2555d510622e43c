"""The reference's PyTorch path for the K8/V4 hot path, restated in torch on the CPU.

TEST INFRASTRUCTURE ONLY (see the package header): this is the CPU baseline
``bench.py`` times on the host cores next to the GPU kernels, and
tests/test_oracle.py checks it against the float64 oracle.  It follows the
reference's own host-side torch code, with torch's intra-op threads:

* store   -- the quantization rule vectorized over (token, head) rows in
             float64 (k8v4_v030/oracle.py:22-69), scales stored as fp32, written
             through strided region views of the page bytes (layout.py:213-256);
* gather  -- block table -> kernel pages, fp32 ``code * k_scale`` and
             ``(nibble - v_zero) * v_scale`` (dequant.py:29-106);
* decode  -- int8-quantized query rows (oracle.py:140-162: the K rule per
             query row), fp32 scores ``dot(q_deq, k_deq) / sqrt(D)``, causal
             ends ``seq_len - q_len + j + 1``, fp32 softmax and P.V;
* prefill -- the key-tiled online-softmax ``eager_prefill`` (dequant.py:160-242,
             :448-501): key tiles of at most 16,384 tokens gathered once each,
             query rows in groups of 256, bottom-right causal mask, fp32.
"""
from __future__ import annotations

import math

import torch

from .paged import PAGE, Geometry

KEY_TILE = 16384
ROW_GROUP = 256
GQA = 6


def region_views(raw: torch.Tensor, geom: Geometry) -> dict[str, torch.Tensor]:
    """Strided views of the five regions of a 1-D uint8 tensor of whole pages."""
    if raw.dtype != torch.uint8 or raw.dim() != 1 or raw.numel() % geom.page_bytes:
        raise ValueError("raw must be a 1-D uint8 tensor of whole pages")
    n, pb, hkv, d = raw.numel() // geom.page_bytes, geom.page_bytes, geom.hkv, geom.d
    off = geom.offsets()
    pages = raw.view(n, pb)

    def region(name, dtype, inner):
        size = {torch.int8: 1, torch.uint8: 1, torch.float32: 4}[dtype]
        nbytes = PAGE * hkv * inner * size
        return pages[:, off[name] : off[name] + nbytes].view(dtype).view(n, PAGE, hkv, inner)

    return {
        "k": region("k", torch.int8, d),
        "v": region("v", torch.uint8, d // 2),
        "k_scale": region("k_scale", torch.float32, 1).squeeze(-1),
        "v_scale": region("v_scale", torch.float32, 1).squeeze(-1),
        "v_zero": region("v_zero", torch.float32, 1).squeeze(-1),
    }


# ----------------------------------------------------------------- store
def quantize_k(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rows ``[..., D]`` -> (int8 codes, float64 scale) under the K rule."""
    x = x.to(torch.float64)
    amax = x.abs().amax(dim=-1)
    scale = amax / 127.0
    inv = torch.where(amax == 0, torch.zeros_like(scale), 1.0 / torch.where(amax == 0, torch.ones_like(scale), scale))
    y = x * inv[..., None]
    code = torch.where(y >= 0, torch.floor(y + 0.5), torch.ceil(y - 0.5)).clamp(-127, 127)
    return code.to(torch.int8), torch.where(amax == 0, torch.zeros_like(scale), scale)


def quantize_v(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Rows ``[..., D]`` -> (packed bytes ``[..., D/2]``, float64 scale, float64 zero)."""
    x = x.to(torch.float64)
    lo, hi = x.amin(dim=-1), x.amax(dim=-1)
    scale = torch.clamp((hi - lo) / 15.0, min=1.0e-8)
    zero = torch.floor(-lo / scale + 0.5).clamp(0, 15)
    code = torch.floor(x / scale[..., None] + zero[..., None] + 0.5).clamp(0, 15).to(torch.uint8)
    return code[..., 0::2] | (code[..., 1::2] << 4), scale, zero


def store(views: dict[str, torch.Tensor], key: torch.Tensor, value: torch.Tensor, slots: torch.Tensor) -> None:
    """Quantize ``[T, hkv, D]`` rows and write token t at ``slots[t]`` (skip slot < 0 or past the cache)."""
    n_pages = views["k"].shape[0]
    slots = slots.to(torch.int64)
    keep = (slots >= 0) & (slots // PAGE < n_pages)
    slots, key, value = slots[keep], key[keep], value[keep]
    page, row = slots // PAGE, slots % PAGE
    k8, ks = quantize_k(key)
    v4, vs, vz = quantize_v(value)
    views["k"][page, row] = k8
    views["k_scale"][page, row] = ks.to(torch.float32)
    views["v"][page, row] = v4
    views["v_scale"][page, row] = vs.to(torch.float32)
    views["v_zero"][page, row] = vz.to(torch.float32)


# ---------------------------------------------------------------- gather
def kernel_pages(block_row: torch.Tensor, page0: int, page1: int, pages_per_block: int) -> torch.Tensor:
    logical = torch.arange(int(page0), int(page1))
    row = block_row.to(torch.int64)
    if int(pages_per_block) == 1:
        return row[logical]
    return row[logical // pages_per_block] * pages_per_block + logical % pages_per_block


def gather_dequant(views, block_row, start: int, end: int, pages_per_block: int = 1):
    """fp32 ``(k, v)`` ``[end - start, hkv, D]`` of tokens ``[start, end)``."""
    p0, p1 = start // PAGE, -(-end // PAGE)
    phys = kernel_pages(block_row, p0, p1, pages_per_block)
    hkv, d = views["k"].shape[2], views["k"].shape[3]
    k = views["k"].index_select(0, phys).to(torch.float32) * views["k_scale"].index_select(0, phys)[..., None]
    packed = views["v"].index_select(0, phys).to(torch.int16)
    vz = views["v_zero"].index_select(0, phys)[..., None]
    vs = views["v_scale"].index_select(0, phys)[..., None]
    v = torch.stack(((packed & 15).to(torch.float32) - vz, (packed >> 4).to(torch.float32) - vz), dim=-1)
    v = (v * vs[..., None]).reshape(-1, hkv, d)
    lo = start - p0 * PAGE
    return k.reshape(-1, hkv, d)[lo : lo + end - start], v[lo : lo + end - start]


# ---------------------------------------------------------------- decode
def decode(views, q: torch.Tensor, block_table: torch.Tensor, seq_lens, q_len: int,
           pages_per_block: int = 1) -> torch.Tensor:
    """``q [B * q_len, HQ, D]`` -> fp32 output, one sequence at a time."""
    hq, d = q.shape[1], q.shape[2]
    hkv = hq // GQA
    out = torch.zeros(q.shape, dtype=torch.float32)
    for b, length in enumerate(int(x) for x in seq_lens):
        if length <= 0:
            continue
        k, v = gather_dequant(views, block_table[b], 0, length, pages_per_block)
        rows = q[b * q_len : (b + 1) * q_len]
        codes, scale = quantize_k(rows)
        qd = (codes.to(torch.float32) * scale.to(torch.float32)[..., None]).view(q_len, hkv, GQA, d)
        scores = torch.einsum("jhgd,thd->hgjt", qd, k) / math.sqrt(d)
        ends = torch.arange(q_len) + (length - q_len + 1)
        dead = torch.arange(length)[None, :] >= ends[:, None]
        scores.masked_fill_(dead[None, None], float("-inf"))
        p = torch.softmax(scores, dim=-1).nan_to_num(0.0)
        out[b * q_len : (b + 1) * q_len] = torch.einsum("hgjt,thd->jhgd", p, v).reshape(q_len, hq, d)
    return out


# --------------------------------------------------------------- prefill
def prefill(views, q: torch.Tensor, block_row: torch.Tensor, seq_len: int, scale: float,
            pages_per_block: int = 1) -> torch.Tensor:
    """``q [q_len, HQ, D]`` (the last q_len tokens) -> fp32 output; key-tiled online softmax."""
    q_len, hq, d = q.shape
    hkv = hq // GQA
    qf = q.to(torch.float32).view(q_len, hkv, GQA, d)
    acc = torch.zeros((hkv, GQA, q_len, d))
    top = torch.full((hkv, GQA, q_len), float("-inf"))
    norm = torch.zeros((hkv, GQA, q_len))
    ends = torch.arange(q_len) + (seq_len - q_len)  # row j sees keys t <= ends[j]
    for k0 in range(0, seq_len, KEY_TILE):
        k1 = min(seq_len, k0 + KEY_TILE)
        k, v = gather_dequant(views, block_row, k0, k1, pages_per_block)
        t = torch.arange(k0, k1)
        for r0 in range(0, q_len, ROW_GROUP):
            r1 = min(q_len, r0 + ROW_GROUP)
            s = torch.einsum("jhgd,thd->hgjt", qf[r0:r1], k) * scale
            s.masked_fill_((t[None, :] > ends[r0:r1, None])[None, None], float("-inf"))
            new_top = torch.maximum(top[:, :, r0:r1], s.amax(dim=-1))
            safe = torch.where(torch.isinf(new_top), torch.zeros_like(new_top), new_top)
            alpha = torch.exp(top[:, :, r0:r1] - safe)
            p = torch.exp(s - safe[..., None])
            norm[:, :, r0:r1] = norm[:, :, r0:r1] * alpha + p.sum(dim=-1)
            acc[:, :, r0:r1] = acc[:, :, r0:r1] * alpha[..., None] + torch.einsum("hgjt,thd->hgjd", p, v)
            top[:, :, r0:r1] = new_top
    return (acc / norm[..., None]).permute(2, 0, 1, 3).reshape(q_len, hq, d)


__all__ = ["decode", "gather_dequant", "kernel_pages", "prefill", "quantize_k", "quantize_v", "region_views",
           "store"]
