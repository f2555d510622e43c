"""Geometry of the int8-K / packed-int4-V paged KV cache.

A kernel page holds 64 consecutive tokens of every local KV head and is
region-major: all K codes first, then all packed V nibbles, then three fp32
planes (K scale, V scale, V zero point).  Within a region the order is
``[token][kv_head][...]``.  A vLLM manager block is a run of whole kernel
pages, so copying one block copies complete pages (prefix caching).

Reference: k8v4_v030/layout.py:16-284.  The reference fixes the head dim at
256; here ``head_dim`` is a field of :class:`PageLayout` (128 or 256) and the
module constant ``D`` keeps the reference default so ``PageLayout(2)`` and
``PageLayout(4)`` mean what they mean there.
"""
from __future__ import annotations

import dataclasses

PAGE = 64
GQA = 6
D = 256
SUPPORTED_HEAD_DIMS = (128, 256)
SUPPORTED_KV_HEADS = (2, 4)
V4_COLS = D // 2
SCALE_BYTES = 4
SLOT_BYTES_PER_HEAD = D + V4_COLS + 3 * SCALE_BYTES
# Rows of one packed decode tile per KV head: q_len * GQA must stay <= 64.
DECODE_MAX_T = PAGE // GQA

CACHE_DTYPE = "int8_k_int4_v"
HISTORIC_MTP_LEN = 59500


def slot_bytes_per_head(head_dim: int) -> int:
    """Bytes one (token, kv_head) pair occupies: D codes, D/2 nibble bytes, 3 floats."""
    head_dim = int(head_dim)
    return head_dim + head_dim // 2 + 3 * SCALE_BYTES


@dataclasses.dataclass(frozen=True)
class PageLayout:
    """Per-rank head layout and the page geometry derived from it.

    ``hkv`` is the number of KV heads this GPU holds (2 for a TP2 rank, 4 when
    one GPU holds all of them); the query side is always ``6 * hkv``.
    """

    hkv: int
    head_dim: int = D

    def __post_init__(self) -> None:
        if self.hkv not in SUPPORTED_KV_HEADS:
            raise ValueError(
                "unsupported per-GPU KV head count %r (K8/V4 serves 2 or 4)" % (self.hkv,)
            )
        if self.head_dim not in SUPPORTED_HEAD_DIMS:
            raise ValueError(
                "unsupported head dim %r (K8/V4 serves %s)" % (self.head_dim, SUPPORTED_HEAD_DIMS)
            )

    @classmethod
    def for_heads(cls, num_heads: int, num_kv_heads: int, head_dim: int = D) -> "PageLayout":
        """Layout for one rank's (query, kv) head pair; anything but 6:1 with 2 or 4 KV fails."""
        nq, nkv = int(num_heads), int(num_kv_heads)
        if nkv not in SUPPORTED_KV_HEADS or nq != GQA * nkv:
            raise ValueError(
                "K8/V4 serves 12/2 (TP2) or 24/4 (single GPU) local heads, got %d Q / %d KV"
                % (nq, nkv)
            )
        return cls(nkv, int(head_dim))

    @property
    def gqa(self) -> int:
        return GQA

    @property
    def hq(self) -> int:
        return GQA * self.hkv

    @property
    def d(self) -> int:
        return self.head_dim

    @property
    def v_cols(self) -> int:
        return self.head_dim // 2

    @property
    def slot_bytes_per_head(self) -> int:
        return slot_bytes_per_head(self.head_dim)

    @property
    def k_bytes_per_page(self) -> int:
        return PAGE * self.hkv * self.head_dim

    @property
    def v_bytes_per_page(self) -> int:
        return PAGE * self.hkv * self.v_cols

    @property
    def scale_bytes_per_page(self) -> int:
        return PAGE * self.hkv * SCALE_BYTES

    @property
    def page_bytes(self) -> int:
        return self.k_bytes_per_page + self.v_bytes_per_page + 3 * self.scale_bytes_per_page

    @property
    def bytes_per_token(self) -> int:
        return self.page_bytes // PAGE

    @property
    def fp8_bytes_per_token(self) -> int:
        """What an fp8 K+V cache would spend on the same heads (2 * D bytes per head)."""
        return 2 * self.hkv * self.head_dim


def pages_per_block(block_size: int) -> int:
    """Kernel pages in one cache block of ``block_size`` tokens."""
    size = int(block_size)
    if size < PAGE or size % PAGE:
        raise ValueError("block_size must be a positive multiple of %d" % PAGE)
    return size // PAGE


def kernel_page_and_offset(slot: int) -> tuple[int, int]:
    """(page, row) a store writes for ``slot``; negative slots map to (-1, -1) and are skipped."""
    s = int(slot)
    if s < 0:
        return -1, -1
    return divmod(s, PAGE)


def n_valid(seq_len: int, logical_page: int) -> int:
    """Tokens of logical page ``logical_page`` that lie below ``seq_len`` (0..64)."""
    left = int(seq_len) - PAGE * int(logical_page)
    return min(PAGE, max(0, left))


def expand_block_ids(block_ids: list[int], ratio: int) -> list[int]:
    """Manager block ids -> kernel page ids (``id * ratio + k`` for k < ratio)."""
    r = int(ratio)
    if r < 1:
        raise ValueError("pages_per_block must be >= 1")
    return [int(b) * r + k for b in block_ids for k in range(r)]


def visible_lens(seq_len: int, q_len: int) -> list[int]:
    """``[max_end, end_0, ..., end_{q-1}]`` for one MTP step.

    Query j (of the last ``q_len`` tokens) sees keys ``t < seq_len - (q_len-1-j)``;
    ends are clamped at 1 and stay full-width integers.
    """
    q, n = int(q_len), int(seq_len)
    if not 1 <= q <= DECODE_MAX_T:
        raise ValueError("q_len %d outside packed decode tile" % q)
    ends = [max(1, n - (q - 1 - j)) for j in range(q)]
    return [max(ends)] + ends


def builtin_q_end(seq_len: int, q_len: int, q_tok: int) -> int:
    """Causal end the kernel derives without ``visible_lens``: seq_len - q_len + q_tok + 1."""
    return int(seq_len) - int(q_len) + int(q_tok) + 1


def as_int16(value: int) -> int:
    """``value`` narrowed to signed 16 bits (the historic length bug, kept for tests)."""
    low = int(value) & 0xFFFF
    return low - 0x10000 if low & 0x8000 else low


def page_regions(page_index: int, layout: PageLayout) -> dict[str, tuple[int, int]]:
    """Byte (offset, length) of the five regions of page ``page_index`` in a packed blob."""
    base = int(page_index) * layout.page_bytes
    sc = layout.scale_bytes_per_page
    k_off = base
    v_off = k_off + layout.k_bytes_per_page
    s_off = v_off + layout.v_bytes_per_page
    return {
        "k": (k_off, layout.k_bytes_per_page),
        "v": (v_off, layout.v_bytes_per_page),
        "k_scale": (s_off, sc),
        "v_scale": (s_off + sc, sc),
        "v_zero": (s_off + 2 * sc, sc),
    }


def block_byte_span(block_id: int, block_size: int, layout: PageLayout) -> tuple[int, int]:
    """(start, length) of one manager block in the packed blob."""
    nbytes = pages_per_block(block_size) * layout.page_bytes
    return int(block_id) * nbytes, nbytes


def attention_pages_per_block(manager_block: int, kernel_block: int | None) -> int:
    """Kernel pages one block-table entry stands for.

    ``kernel_block is None`` means the table still holds manager blocks.  A
    64-token kernel block is one page; a wider one expands as
    ``entry * ratio + page_in_entry``, the same page ``slot // 64`` writes.
    """
    mb = int(manager_block)
    if mb < PAGE or mb % PAGE:
        raise ValueError("manager block %s is not a multiple of %s" % (mb, PAGE))
    if kernel_block is None:
        return mb // PAGE
    kb = int(kernel_block)
    if kb < PAGE or kb % PAGE:
        raise ValueError("kernel block %s is not a multiple of %s" % (kb, PAGE))
    return kb // PAGE


def table_block_size(manager_block: int, kernel_block: int | None) -> int:
    """Tokens covered by one block-table entry."""
    return int(manager_block) if kernel_block is None else int(kernel_block)


def max_kernel_pages(max_model_len: int, manager_block: int, kernel_block: int | None) -> int:
    """Kernel pages a full-length block-table row can address."""
    unit = table_block_size(manager_block, kernel_block)
    ratio = attention_pages_per_block(manager_block, kernel_block)
    entries = max(1, -(-int(max_model_len) // unit))
    return entries * ratio


_ELEM_BYTES = {"int8": 1, "uint8": 1, "float32": 4}


def region_view_specs(num_pages: int, layout: PageLayout) -> dict[str, dict[str, object]]:
    """``as_strided`` specs (shape, element stride, byte offset) of the five regions.

    The page stride of every region is one whole page, so consecutive pages of
    one region are not adjacent.
    """
    n = int(num_pages)
    if n < 1:
        raise ValueError("num_pages")
    d, hkv, pb = layout.head_dim, layout.hkv, layout.page_bytes
    scale0 = layout.k_bytes_per_page + layout.v_bytes_per_page
    fstride = pb // SCALE_BYTES
    plane = {
        "dtype": "float32",
        "shape": (n, PAGE, hkv),
        "stride": (fstride, hkv, 1),
    }
    return {
        "k": {
            "dtype": "int8",
            "shape": (n, PAGE, hkv, d),
            "stride": (pb, hkv * d, d, 1),
            "byte_offset": 0,
        },
        "v": {
            "dtype": "uint8",
            "shape": (n, PAGE, hkv, d // 2),
            "stride": (pb, hkv * (d // 2), d // 2, 1),
            "byte_offset": layout.k_bytes_per_page,
        },
        "k_scale": dict(plane, byte_offset=scale0),
        "v_scale": dict(plane, byte_offset=scale0 + layout.scale_bytes_per_page),
        "v_zero": dict(plane, byte_offset=scale0 + 2 * layout.scale_bytes_per_page),
    }


def element_byte(spec: dict[str, object], index: tuple[int, ...]) -> int:
    """Byte address (from page 0) of one element of a region spec; bounds-checked."""
    shape, stride = spec["shape"], spec["stride"]
    if len(index) != len(shape) or len(stride) != len(shape):
        raise ValueError("index rank")
    elem = _ELEM_BYTES[str(spec["dtype"])]
    addr = int(spec["byte_offset"])
    for i, size, step in zip(index, shape, stride):
        i = int(i)
        if not 0 <= i < int(size):
            raise IndexError(i)
        addr += i * int(step) * elem
    return addr


def region_stays_inside_block(block_size: int, layout: PageLayout) -> bool:
    """True when every region of every page of block 0 lies inside that block's bytes."""
    start, length = block_byte_span(0, block_size, layout)
    end = start + length
    for page in range(pages_per_block(block_size)):
        for off, nbytes in page_regions(page, layout).values():
            if off < start or off + nbytes > end:
                return False
    return True
