"""Writes the committed golden fixtures of this directory.

1. ``quant_known_answers.json`` -- rows whose expected codes follow by hand
   from the reference quantization rule (k8v4_v030/oracle.py:18-69).  Every
   row uses values exactly representable in fp16 and scales that are powers
   of two, so the expected codes need no floating-point reasoning beyond the
   rounding rule itself.  The derivation of each expectation is written next
   to it.  Rows are zero-padded to the head dim.
2. ``reference_geometry.json`` -- constants the reference's own tests pin
   (k8v4_v030/tests/test_layout_mtp.py:50-78, :105-143, :176-200 and
   test_plan_scratch.py:44-58), plus the D=128 page geometry the build's
   configs use (204 bytes per token and KV head, 52,224-byte pages at 4 heads).

Run: ``python tests/golden/make_fixtures.py`` (rewrites both files).
"""
from __future__ import annotations

import json
from pathlib import Path

HERE = Path(__file__).resolve().parent

# ---- K rule: amax/127 scale, half-away-from-zero rounding, clamp +-127 ----
K_CASES = [
    {
        "name": "k_ties_scale_one",
        # amax 127 -> scale 1, inv 1: y == x.  x.5 ties round away from zero
        # (round-half-even would give 2, -2, 0, 0, 2 for the first five ties).
        "values": [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 126.5, -126.5, 3.25, -3.75],
        "codes": [127, 3, -3, 1, -1, 2, 127, -127, 3, -4],
        "scale": 1.0,
    },
    {
        "name": "k_ties_scale_1_128",
        # amax 127/128 -> scale 1/128, inv 128: y = 128 x.
        # 3/256 -> 1.5 -> 2; 5/256 -> 2.5 -> 3; -5/256 -> -3; 1/256 -> 0.5 -> 1.
        "values": [0.9921875, 0.01171875, 0.01953125, -0.01953125, 0.00390625, -0.9921875],
        "codes": [127, 2, 3, -3, 1, -127],
        "scale": 0.0078125,
    },
    {
        "name": "k_zero_row",
        # amax 0: every code 0 and the stored scale is 0.
        "values": [0.0],
        "codes": [0],
        "scale": 0.0,
    },
]

# ---- V rule: affine 4-bit, scale max((hi-lo)/15, 1e-8), floor(x+0.5) ----
V_CASES = [
    {
        "name": "v_ties_lo0_hi15",
        # lo 0, hi 15 -> scale 1, zero floor(0.5) = 0; code floor(x + 0.5):
        # 2.5 -> 3, 7.5 -> 8, 14.5 -> 15, 0.5 -> 1, 15 -> floor(15.5) = 15,
        # 1.25 -> 1, 1.75 -> 2 (round-half-even would give 2, 8, 14, 0 for the ties).
        "values": [2.5, 7.5, 14.5, 0.5, 15.0, 1.25, 1.75, 0.0],
        "nibbles": [3, 8, 15, 1, 15, 1, 2, 0],
        "scale": 1.0,
        "zero": 0.0,
    },
    {
        "name": "v_signed_span",
        # lo -7.5, hi 7.5 -> scale 1, zero floor(7.5 + 0.5) = 8;
        # -7.5 -> 1, 7.5 -> floor(16) clamped 15, 0 -> 8, -2.5 -> 6, 2.5 -> 11.
        "values": [-7.5, 7.5, 0.0, -2.5, 2.5],
        "nibbles": [1, 15, 8, 6, 11],
        "scale": 1.0,
        "zero": 8.0,
    },
    {
        "name": "v_constant_positive",
        # hi == lo: scale 1e-8; zero floor(-0.5e8 + 0.5) clamps to 0; every code
        # floor(0.5e8 + 0.5) clamps to 15.  (Padding is 0.5 too: a constant row.)
        "values": [0.5],
        "pad": 0.5,
        "nibbles": [15],
        "scale": 1.0e-8,
        "zero": 0.0,
    },
    {
        "name": "v_constant_negative",
        # zero floor(0.5e8 + 0.5) clamps to 15; codes floor(-0.5e8 + 15.5) clamp to 0.
        "values": [-0.5],
        "pad": -0.5,
        "nibbles": [0],
        "scale": 1.0e-8,
        "zero": 15.0,
    },
    {
        "name": "v_zero_row",
        # 0/1e-8 + 0 + 0.5 -> code 0; zero floor(0.5) = 0.
        "values": [0.0],
        "nibbles": [0],
        "scale": 1.0e-8,
        "zero": 0.0,
    },
]

GEOMETRY = {
    "source": "k8v4_v030/tests/test_layout_mtp.py:50-78,105-143,176-200; test_plan_scratch.py:44-58",
    "slot_bytes_per_head_d256": 396,
    "d256": {
        "hkv2": {"bytes_per_token": 792, "page_bytes": 50688, "fp8_bytes_per_token": 1024},
        "hkv4": {"bytes_per_token": 1584, "page_bytes": 101376, "fp8_bytes_per_token": 2048},
    },
    "d128": {
        "slot_bytes_per_head": 204,
        "hkv4": {
            "bytes_per_token": 816,
            "page_bytes": 52224,
            "regions": {"k": 32768, "v": 16384, "k_scale": 1024, "v_scale": 1024, "v_zero": 1024},
        },
    },
    "attention_pages_per_block": [[1664, 64, 1], [1664, None, 26], [2112, 2112, 33],
                                  [2112, None, 33], [2112, 64, 1], [1664, 1664, 26]],
    "max_kernel_pages": [[131072, 1664, 64, 2048], [131072, 1664, None, 2054],
                         [131072, 1664, 1664, 2054]],
    "kernel_page_and_offset": [[-1, -1, -1], [0, 0, 0], [63, 0, 63], [64, 1, 0], [454, 7, 6]],
    "n_valid": [[63, 0, 63], [64, 0, 64], [65, 1, 1], [59500, 929, 44], [59500, 930, 0]],
    "expand_block_ids": {"ids": [3, 5], "ratio": 2, "pages": [6, 7, 10, 11]},
    "visible_lens_59500_q7": [59500, 59494, 59495, 59496, 59497, 59498, 59499, 59500],
    "as_int16_59500": -6036,
    "scratch_capacity": {
        "args": [131072, 1664, 1664, 8192, 8, [7, 14, 21, 28, 35, 42, 49, 56]],
        "nprog_per_hkv": 2080, "store": 8192, "out": 80,
        "split_64_nprog_per_hkv": 2049,
    },
}


def main() -> None:
    (HERE / "quant_known_answers.json").write_text(
        json.dumps({"rule": "k8v4_v030/oracle.py:18-69", "k": K_CASES, "v": V_CASES}, indent=1) + "\n"
    )
    (HERE / "reference_geometry.json").write_text(json.dumps(GEOMETRY, indent=1) + "\n")


if __name__ == "__main__":
    main()
