"""Pure-Python scalar restatement of the reference oracle, for tiny inputs.

Reference: k8v4_v030/oracle.py:18-174.  Plain Python floats are IEEE doubles,
so this file and ``oracle.quant`` must agree bit for bit; the test suite checks
that on random and adversarial rows.  ``causal_gqa`` here follows
oracle.py:100-163: K/V and every Q row are quantized with the store rule, the
score is the exact integer dot times the two (double) scales over sqrt(D), the
mask ends query j at ``seq_len - q_len + j + 1``, softmax is float64 (a row
with no visible key returns zeros) and V is dequantized in double.  Unlike the
reference it takes the head dim from the rows instead of fixing 256.
"""
from __future__ import annotations

import math
import random

GQA = 6


def rint_half_away(value: float) -> int:
    return int(math.floor(value + 0.5)) if value >= 0 else int(math.ceil(value - 0.5))


def quant_k(row: list[float]) -> tuple[list[int], float]:
    amax = 0.0
    for v in row:
        amax = max(amax, abs(v))
    if amax == 0.0:
        return [0] * len(row), 0.0
    scale = amax / 127.0
    inv = 1.0 / scale
    out = []
    for v in row:
        out.append(min(127, max(-127, rint_half_away(v * inv))))
    return out, scale


def quant_v(row: list[float]) -> tuple[list[int], float, float]:
    lo, hi = min(row), max(row)
    scale = max((hi - lo) / 15.0, 1.0e-8)
    zero = min(15, max(0, math.floor(-lo / scale + 0.5)))
    nib = [min(15, max(0, math.floor(v / scale + zero + 0.5))) for v in row]
    packed = [nib[i] | (nib[i + 1] << 4) for i in range(0, len(row), 2)]
    return packed, scale, float(zero)


def dequant_v(packed: list[int], scale: float, zero: float) -> list[float]:
    out = []
    for b in packed:
        out.append((float(b & 0xF) - zero) * scale)
        out.append((float(b >> 4) - zero) * scale)
    return out


def softmax(scores: list[float]) -> list[float]:
    live = [s for s in scores if s != float("-inf")]
    if not live:
        return [0.0] * len(scores)
    top = max(live)
    ex = [0.0 if s == float("-inf") else math.exp(s - top) for s in scores]
    total = sum(ex)
    if total == 0.0:
        return [0.0] * len(scores)
    return [e / total for e in ex]


def causal_gqa(query, key, value, seq_len: int, q_len: int):
    """query ``[q_len][HQ][D]``, key/value ``[>=seq_len][HKV][D]`` -> ``[q_len][HQ][D]``."""
    if len(query) != q_len:
        raise ValueError("query width")
    if len(key) < seq_len or len(value) < seq_len:
        raise ValueError("cache shorter than seq_len")
    if q_len == 0:
        return []
    hq = len(query[0])
    d = len(query[0][0])
    hkv = len(key[0]) if key else hq // GQA
    if hq != GQA * hkv:
        raise ValueError("head pair")
    kq = [[quant_k(key[t][h]) for h in range(hkv)] for t in range(seq_len)]
    vq = [[dequant_v(*quant_v(value[t][h])) for h in range(hkv)] for t in range(seq_len)]
    inv_sqrt = 1.0 / math.sqrt(d)
    out = []
    for j in range(q_len):
        end = seq_len - q_len + j + 1
        heads = []
        for h in range(hq):
            g = h // GQA
            qc, qs = quant_k(query[j][h])
            scores = []
            for t in range(seq_len):
                if t >= end:
                    scores.append(float("-inf"))
                    continue
                kc, ks = kq[t][g]
                dot = sum(a * b for a, b in zip(qc, kc))
                scores.append(dot * qs * ks * inv_sqrt)
            probs = softmax(scores)
            acc = [0.0] * d
            for t, p in enumerate(probs):
                if p == 0.0:
                    continue
                row = vq[t][g]
                for i in range(d):
                    acc[i] += p * row[i]
            heads.append(acc)
        out.append(heads)
    return out


def deterministic_rows(n: int, heads: int, seed: int, dim: int = 256):
    """``[n][heads][dim]`` uniform(-1, 1) rows from ``random.Random(seed)`` (oracle.py:166-174)."""
    rng = random.Random(seed)
    return [[[rng.uniform(-1.0, 1.0) for _ in range(dim)] for _ in range(heads)] for _ in range(n)]
