"""Vectorized float64 restatement of the K8/V4 quantization rule.

Reference: k8v4_v030/oracle.py:18-77 (``_rint``, ``quant_k``, ``dequant_k``,
``quant_v``, ``dequant_v``) and the fp32 storage of scales in
k8v4_v030/paged.py:56-65 (``struct.pack('<f', x)``: round-to-nearest-even from
double).  Every arithmetic step is the same IEEE double operation in the same
order as the reference's Python floats, so codes are bit-identical:

* K: ``amax = max|x|``; amax == 0 -> codes 0, scale 0.  Else
  ``scale = amax / 127``, ``inv = 1 / scale``, ``y = x * inv`` and the code is
  ``floor(y + 0.5)`` for y >= 0, ``ceil(y - 0.5)`` for y < 0 (half away from
  zero), clamped to [-127, 127].
* V: ``lo = min x``, ``hi = max x``, ``scale = max((hi - lo) / 15, 1e-8)``,
  ``zero = clamp(floor(-lo / scale + 0.5), 0, 15)``, code
  ``clamp(floor(x / scale + zero + 0.5), 0, 15)``; byte ``i`` packs dims
  ``2i`` (low nibble) and ``2i+1`` (high nibble).
"""
from __future__ import annotations

import numpy as np


def quant_k(rows) -> tuple[np.ndarray, np.ndarray]:
    """``rows[..., D]`` -> (int8 codes ``[..., D]``, float64 scale ``[...]``)."""
    x = np.asarray(rows, dtype=np.float64)
    amax = np.max(np.abs(x), axis=-1)
    zero_row = amax == 0.0
    scale = amax / 127.0
    inv = 1.0 / np.where(zero_row, 1.0, scale)
    y = x * inv[..., None]
    code = np.where(y >= 0.0, np.floor(y + 0.5), np.ceil(y - 0.5))
    code = np.clip(code, -127.0, 127.0)
    code[zero_row] = 0.0
    scale = np.where(zero_row, 0.0, scale)
    return code.astype(np.int8), scale


def dequant_k(codes, scale) -> np.ndarray:
    """float64 ``code * scale`` (oracle.py:43-44)."""
    return np.asarray(codes, dtype=np.float64) * np.asarray(scale, dtype=np.float64)[..., None]


def quant_v_nibbles(rows) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``rows[..., D]`` -> (nibbles uint8 ``[..., D]`` in 0..15, scale f64, zero f64)."""
    x = np.asarray(rows, dtype=np.float64)
    lo = np.min(x, axis=-1)
    hi = np.max(x, axis=-1)
    scale = np.maximum((hi - lo) / 15.0, 1.0e-8)
    zero = np.clip(np.floor(-lo / scale + 0.5), 0.0, 15.0)
    code = np.floor(x / scale[..., None] + zero[..., None] + 0.5)
    code = np.clip(code, 0.0, 15.0)
    return code.astype(np.uint8), scale, zero


def pack_nibbles(nib: np.ndarray) -> np.ndarray:
    """``[..., D]`` nibbles -> ``[..., D/2]`` bytes, low nibble = even dim."""
    nib = np.asarray(nib, dtype=np.uint8)
    return (nib[..., 0::2] | (nib[..., 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """``[..., D/2]`` bytes -> ``[..., D]`` nibbles (inverse of :func:`pack_nibbles`)."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (2 * packed.shape[-1],), dtype=np.uint8)
    out[..., 0::2] = packed & 0x0F
    out[..., 1::2] = packed >> 4
    return out


def quant_v(rows) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``rows[..., D]`` -> (packed bytes ``[..., D/2]``, scale f64, zero f64)."""
    nib, scale, zero = quant_v_nibbles(rows)
    return pack_nibbles(nib), scale, zero


def dequant_v(packed, scale, zero) -> np.ndarray:
    """float64 ``(nibble - zero) * scale`` (oracle.py:72-77)."""
    nib = unpack_nibbles(packed).astype(np.float64)
    z = np.asarray(zero, dtype=np.float64)[..., None]
    s = np.asarray(scale, dtype=np.float64)[..., None]
    return (nib - z) * s


def stored_f32(values) -> np.ndarray:
    """The fp32 a scale/zero is stored as: IEEE round-to-nearest-even from double."""
    return np.asarray(values, dtype=np.float64).astype(np.float32)
