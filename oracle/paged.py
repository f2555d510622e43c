"""The K8/V4 page byte format, slot store and block-table gather, on a numpy byte blob.

Reference:
* page geometry and region order -- k8v4_v030/layout.py:67-89, :153-165, :213-256;
* byte-level token pack/unpack   -- k8v4_v030/paged.py:30-91 (``write_token`` /
  ``read_token``; scales stored as little-endian fp32);
* store skip rule                -- native/xe2_kv_ops.cpp:549-563 (slot < 0 or
  page >= num_pages writes nothing);
* logical -> physical page map   -- dequant.py:40-55 (``bt[p]`` when one table
  entry is one page, else ``bt[p // r] * r + p % r``);
* dequant                         -- dequant.py:96-106 (fp32 ``code * k_scale``
  and ``(nibble - v_zero) * v_scale``).

The geometry is computed here from first principles, not imported from the
product package, so the product's layout code is checked against it.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from . import quant

PAGE = 64


@dataclass(frozen=True)
class Geometry:
    hkv: int
    d: int

    @property
    def k_bytes(self) -> int:  # [64][hkv][d] int8
        return PAGE * self.hkv * self.d

    @property
    def v_bytes(self) -> int:  # [64][hkv][d/2] packed nibbles
        return PAGE * self.hkv * self.d // 2

    @property
    def plane_bytes(self) -> int:  # [64][hkv] fp32
        return PAGE * self.hkv * 4

    @property
    def page_bytes(self) -> int:
        return self.k_bytes + self.v_bytes + 3 * self.plane_bytes

    def offsets(self) -> dict[str, int]:
        """Byte offset of each region inside a page."""
        s0 = self.k_bytes + self.v_bytes
        return {
            "k": 0,
            "v": self.k_bytes,
            "k_scale": s0,
            "v_scale": s0 + self.plane_bytes,
            "v_zero": s0 + 2 * self.plane_bytes,
        }


def new_blob(num_pages: int, geom: Geometry, fill: int = 0) -> np.ndarray:
    return np.full(int(num_pages) * geom.page_bytes, fill, dtype=np.uint8)


def regions(blob: np.ndarray, geom: Geometry) -> dict[str, np.ndarray]:
    """Strided numpy views of the five regions (writes go through to ``blob``)."""
    if blob.dtype != np.uint8 or blob.ndim != 1 or blob.size % geom.page_bytes:
        raise ValueError("blob must be a 1-D uint8 array of whole pages")
    n = blob.size // geom.page_bytes
    pb, hkv, d = geom.page_bytes, geom.hkv, geom.d
    off = geom.offsets()
    buf = blob.data

    def view(dtype, shape, strides, offset):
        return np.ndarray(shape, dtype=dtype, buffer=buf, offset=offset, strides=strides)

    plane = ((n, PAGE, hkv), (pb, hkv * 4, 4))
    return {
        "k": view(np.int8, (n, PAGE, hkv, d), (pb, hkv * d, d, 1), off["k"]),
        "v": view(np.uint8, (n, PAGE, hkv, d // 2), (pb, hkv * d // 2, d // 2, 1), off["v"]),
        "k_scale": view(np.float32, *plane, off["k_scale"]),
        "v_scale": view(np.float32, *plane, off["v_scale"]),
        "v_zero": view(np.float32, *plane, off["v_zero"]),
    }


def store(blob: np.ndarray, geom: Geometry, key, value, slots) -> None:
    """Quantize ``key``/``value`` ``[T, hkv, d]`` and write token t at ``slots[t]``.

    Invalid slots (negative, or past the last page) are skipped entirely.
    """
    key = np.asarray(key, dtype=np.float64)
    value = np.asarray(value, dtype=np.float64)
    slots = np.asarray(slots, dtype=np.int64)
    r = regions(blob, geom)
    num_pages = r["k"].shape[0]
    page = np.where(slots >= 0, slots // PAGE, -1)
    ok = (slots >= 0) & (page < num_pages)
    if not ok.any():
        return
    kc, ks = quant.quant_k(key[ok])
    vp, vs, vz = quant.quant_v(value[ok])
    p, row = page[ok], slots[ok] % PAGE
    r["k"][p, row] = kc
    r["k_scale"][p, row] = quant.stored_f32(ks)
    r["v"][p, row] = vp
    r["v_scale"][p, row] = quant.stored_f32(vs)
    r["v_zero"][p, row] = quant.stored_f32(vz)


def _byte_addr(geom: Geometry, page: int, row: int, head: int, region: str, col: int = 0) -> int:
    """Address arithmetic written out longhand (independent of the strided views)."""
    base = page * geom.page_bytes + geom.offsets()[region]
    if region == "k":
        return base + (row * geom.hkv + head) * geom.d + col
    if region == "v":
        return base + (row * geom.hkv + head) * (geom.d // 2) + col
    return base + (row * geom.hkv + head) * 4


def write_token(blob: np.ndarray, geom: Geometry, slot: int, keys, values) -> None:
    """Byte-level store of one token (``keys``/``values`` are ``[hkv][d]``); slot < 0 is a no-op."""
    if slot < 0:
        return
    page, row = divmod(int(slot), PAGE)
    if (page + 1) * geom.page_bytes > blob.size:
        raise ValueError("blob shorter than page %d" % page)
    for h in range(geom.hkv):
        codes, ks = quant.quant_k(np.asarray(keys[h], dtype=np.float64)[None])
        a = _byte_addr(geom, page, row, h, "k")
        blob[a : a + geom.d] = codes[0].view(np.uint8)
        a = _byte_addr(geom, page, row, h, "k_scale")
        blob[a : a + 4] = np.frombuffer(struct.pack("<f", float(ks[0])), dtype=np.uint8)
        packed, vs, vz = quant.quant_v(np.asarray(values[h], dtype=np.float64)[None])
        a = _byte_addr(geom, page, row, h, "v")
        blob[a : a + geom.d // 2] = packed[0]
        for name, val in (("v_scale", vs[0]), ("v_zero", vz[0])):
            a = _byte_addr(geom, page, row, h, name)
            blob[a : a + 4] = np.frombuffer(struct.pack("<f", float(val)), dtype=np.uint8)


def read_token(blob: np.ndarray, geom: Geometry, slot: int):
    """Inverse of :func:`write_token` up to rounding: (keys ``[hkv][d]``, values ``[hkv][d]``)."""
    if slot < 0:
        raise ValueError("negative slot")
    page, row = divmod(int(slot), PAGE)
    keys, values = [], []
    for h in range(geom.hkv):
        a = _byte_addr(geom, page, row, h, "k")
        codes = blob[a : a + geom.d].view(np.int8).astype(np.float64)
        a = _byte_addr(geom, page, row, h, "k_scale")
        (ks,) = struct.unpack("<f", blob[a : a + 4].tobytes())
        keys.append(codes * ks)
        a = _byte_addr(geom, page, row, h, "v")
        packed = blob[a : a + geom.d // 2].copy()
        fl = []
        for name in ("v_scale", "v_zero"):
            a = _byte_addr(geom, page, row, h, name)
            fl.append(struct.unpack("<f", blob[a : a + 4].tobytes())[0])
        values.append(quant.dequant_v(packed, fl[0], fl[1]))
    return keys, values


def physical_pages(block_row, page0: int, page1: int, pages_per_block: int) -> np.ndarray:
    """Physical kernel pages of logical pages ``[page0, page1)``."""
    row = np.asarray(block_row, dtype=np.int64)
    r = int(pages_per_block)
    if r < 1:
        raise ValueError("pages_per_block")
    logical = np.arange(int(page0), int(page1), dtype=np.int64)
    if r == 1:
        return row[logical]
    return row[logical // r] * r + logical % r


def gather_codes(blob, geom: Geometry, block_row, start: int, end: int, pages_per_block: int):
    """Codes and fp32 planes of tokens ``[start, end)``: k8, k_scale, v nibbles, v_scale, v_zero."""
    r = regions(blob, geom)
    n = max(0, int(end) - int(start))
    if n == 0:
        z = np.zeros((0, geom.hkv), np.float32)
        return (np.zeros((0, geom.hkv, geom.d), np.int8), z,
                np.zeros((0, geom.hkv, geom.d), np.uint8), z, z)
    p0, p1 = start // PAGE, (end + PAGE - 1) // PAGE
    phys = physical_pages(block_row, p0, p1, pages_per_block)
    lo = start - p0 * PAGE
    sl = slice(lo, lo + n)
    k8 = r["k"][phys].reshape(-1, geom.hkv, geom.d)[sl]
    ks = r["k_scale"][phys].reshape(-1, geom.hkv)[sl]
    vn = quant.unpack_nibbles(r["v"][phys]).reshape(-1, geom.hkv, geom.d)[sl]
    vs = r["v_scale"][phys].reshape(-1, geom.hkv)[sl]
    vz = r["v_zero"][phys].reshape(-1, geom.hkv)[sl]
    return k8, ks, vn, vs, vz


def dequant_f32(k8, ks, vn, vs, vz) -> tuple[np.ndarray, np.ndarray]:
    """fp32 K and V exactly as the reference's torch gather computes them."""
    k = k8.astype(np.float32) * ks.astype(np.float32)[..., None]
    v = (vn.astype(np.float32) - vz.astype(np.float32)[..., None]) * vs.astype(np.float32)[..., None]
    return k, v


def gather_dequant(blob, geom: Geometry, block_row, seq_len: int, pages_per_block: int,
                   start: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """fp32 ``(k, v)`` shaped ``[seq_len - start, hkv, d]``."""
    return dequant_f32(*gather_codes(blob, geom, block_row, start, seq_len, pages_per_block))
