"""Process-wide, capture-stable decode scratch (one per device and layout).

Buffers are allocated before graph capture; forward only narrows them, so a
captured launch keeps stable addresses.  Reference: k8v4_v030/scratch.py:17-115
(same fields and reuse rules).  The q8/q_scale/merged tensors keep their
reference shapes for callers that pass them; the decode kernel here quantizes
Q in its prologue and uses the ``partials`` bytes as its split-K state.
"""
from __future__ import annotations

import torch

from .layout import PAGE, PageLayout

_SLOTS: dict[tuple[str, int | None, int, int], "Scratch"] = {}


class Scratch:
    def __init__(
        self,
        device: torch.device,
        layout: PageLayout,
        nprog_max: int,
        max_store_tokens: int,
        max_out_tokens: int,
    ):
        if nprog_max < 1 or max_store_tokens < 1 or max_out_tokens < 1:
            raise ValueError("scratch capacity")
        self.device = device
        self.layout = layout
        self.nprog_max = int(nprog_max)
        self.max_store_tokens = int(max_store_tokens)
        self.max_out_tokens = int(max_out_tokens)
        hkv, hq, d = layout.hkv, layout.hq, layout.head_dim
        f32 = dict(dtype=torch.float32, device=device)
        f16 = dict(dtype=torch.float16, device=device)
        self.q8 = torch.empty((hkv, PAGE, d), dtype=torch.int8, device=device)
        self.q_scale = torch.empty((hkv, PAGE), **f32)
        self.k_fp16 = torch.empty((self.max_store_tokens, hkv, d), **f16)
        self.v_fp16 = torch.empty((self.max_store_tokens, hkv, d), **f16)
        self.q_fp16 = torch.empty((self.max_out_tokens, hq, d), **f16)
        self.out_fp16 = torch.empty((self.max_out_tokens, hq, d), **f16)
        self.partials = torch.empty((self.nprog_max, PAGE, d), **f32)
        self.m = torch.empty((self.nprog_max, PAGE), **f32)
        self.l = torch.empty((self.nprog_max, PAGE), **f32)
        self.merged = torch.empty((hkv, PAGE, d), **f32)
        # numel 0 means "derive the causal ends from seq_lens".
        self.visible = torch.empty((0,), dtype=torch.int32, device=device)

    def workspace(self, nprog: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        n = int(nprog)
        if not 1 <= n <= self.nprog_max:
            raise RuntimeError(
                "K8/V4 workspace needs %d programs and was allocated for %d" % (n, self.nprog_max)
            )
        return self.partials[:n], self.m[:n], self.l[:n], self.merged

    def store_pair(self, ntok: int) -> tuple[torch.Tensor, torch.Tensor]:
        n = int(ntok)
        if not 1 <= n <= self.max_store_tokens:
            raise RuntimeError(
                "K8/V4 store buffer holds %d tokens, got %d" % (self.max_store_tokens, n)
            )
        return self.k_fp16[:n], self.v_fp16[:n]

    def attention_pair(self, ntok: int) -> tuple[torch.Tensor, torch.Tensor]:
        n = int(ntok)
        if not 1 <= n <= self.max_out_tokens:
            raise RuntimeError(
                "K8/V4 attention buffer holds %d tokens, got %d" % (self.max_out_tokens, n)
            )
        return self.q_fp16[:n], self.out_fp16[:n]


def scratch_key(device: torch.device, layout: PageLayout) -> tuple[str, int | None, int, int]:
    device = torch.device(device)
    index = device.index
    if index is None and device.type == "cuda":
        index = torch.cuda.current_device()  # "cuda" and "cuda:N" name the same slot
    return (device.type, index, layout.hkv, layout.head_dim)


def ensure_scratch(
    device: torch.device,
    layout: PageLayout,
    nprog_max: int,
    max_store_tokens: int,
    max_out_tokens: int,
) -> Scratch:
    """The cached scratch for (device, layout) if it is big enough, else a new, larger one."""
    key = scratch_key(device, layout)
    have = _SLOTS.get(key)
    if (
        have is not None
        and have.nprog_max >= int(nprog_max)
        and have.max_store_tokens >= int(max_store_tokens)
        and have.max_out_tokens >= int(max_out_tokens)
    ):
        return have
    have = Scratch(device, layout, nprog_max, max_store_tokens, max_out_tokens)
    _SLOTS[key] = have
    return have


def get_scratch(device: torch.device, layout: PageLayout) -> Scratch:
    key = scratch_key(device, layout)
    if key not in _SLOTS:
        raise RuntimeError("K8/V4 scratch was not allocated before attention")
    return _SLOTS[key]


def scratch_ready(device: torch.device, layout: PageLayout) -> bool:
    return scratch_key(device, layout) in _SLOTS


def clear_scratch() -> None:
    _SLOTS.clear()
