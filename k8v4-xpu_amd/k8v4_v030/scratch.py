"""Device buffers the K8/V4 kernels write besides the cache, one set per (device, layout).

The HIP library needs exactly two scratch buffers, both caller-owned so that
a captured HIP graph keeps stable addresses and no call allocates:

* the decode workspace -- split-K states of ``k8v4_attn_batch`` (fp16 partial
  outputs plus fp32 max / sum per split, head and query row), sized by the
  library (``k8v4_attn_workspace_bytes``) for the widest decode call the
  engine can issue;
* the prefill workspace -- partial softmax states of the row blocks that
  ``k8v4_prefill_paged`` splits between work-groups, sized by the library
  (``k8v4_prefill_workspace_bytes``) for the longest chunk over the longest
  context, and at least what one launch of ``k8v4_prefill_paged_batch``
  (a step's short chunks together) needs.

Capacity is given in the reference's terms (k8v4_v030/scratch.py:17-115):
``nprog_max`` = kernel pages of the longest sequence times the KV head count,
``max_store_tokens`` = tokens one step may store (the longest prefill chunk),
``max_out_tokens`` = query tokens of the widest decode call.  The reference
also keeps fp16 staging copies, an int8 query tile and fp32 per-page
partials; the kernels here take vLLM's rows in place, quantize the query in
the decode prologue and keep their split states in the decode workspace, so
those buffers exist only as lazily created objects for callers that still
ask for them (``q8``, ``q_scale``, ``store_pair``, ``attention_pair``).
"""
from __future__ import annotations

import torch

from .layout import DECODE_MAX_T, PAGE, PageLayout

_REGISTRY: dict[tuple[str, int | None, int, int], "Scratch"] = {}


def _library_ops():
    from .ops_api import ops

    return ops()


def decode_workspace_bytes(layout: PageLayout, max_pages: int, max_out_tokens: int,
                           max_seqs: int | None = None) -> int:
    """Largest decode workspace over every query length 1..10 at ``max_out_tokens``
    query rows, for at most ``max_seqs`` sequences per call (when given: a
    decode call never holds more sequences than the engine schedules, however
    many query rows the output buffer allows)."""
    lib = _library_ops()
    need = 0
    for q_len in range(1, DECODE_MAX_T + 1):
        batch = max(1, int(max_out_tokens) // q_len)
        if max_seqs is not None:
            batch = max(1, min(batch, int(max_seqs)))
        need = max(need, lib.attn_workspace_bytes(batch, int(max_pages), 1, q_len, layout.hkv, layout.head_dim))
    return need


def prefill_workspace_bytes(layout: PageLayout, max_pages: int, max_chunk: int) -> int:
    """Prefill workspace for a ``max_chunk``-token query over ``max_pages`` pages of
    context, and for a batch of a step's short chunks in one call."""
    seq_len = int(max_pages) * PAGE
    chunk = max(1, min(int(max_chunk), seq_len))
    lib = _library_ops()
    return max(lib.prefill_workspace_bytes(seq_len, chunk, layout.hkv, layout.head_dim),
               lib.prefill_batch_workspace_bytes(layout.hkv, layout.head_dim))


class Scratch:
    """The decode and prefill workspaces of one device and head layout."""

    def __init__(
        self,
        device: torch.device,
        layout: PageLayout,
        nprog_max: int,
        max_store_tokens: int,
        max_out_tokens: int,
        max_seqs: int | None = None,
    ):
        if min(int(nprog_max), int(max_store_tokens), int(max_out_tokens)) < 1:
            raise ValueError("scratch capacity")
        if max_seqs is not None and int(max_seqs) < 1:
            raise ValueError("scratch capacity")
        self.device = torch.device(device)
        self.layout = layout
        self.nprog_max = int(nprog_max)
        self.max_store_tokens = int(max_store_tokens)
        self.max_out_tokens = int(max_out_tokens)
        self.max_seqs = None if max_seqs is None else int(max_seqs)
        self.max_pages = -(-self.nprog_max // layout.hkv)
        self.decode_bytes = decode_workspace_bytes(layout, self.max_pages, self.max_out_tokens, self.max_seqs)
        self.prefill_bytes = prefill_workspace_bytes(layout, self.max_pages, self.max_store_tokens)
        self.decode_ws = torch.empty(_words(self.decode_bytes), dtype=torch.int32, device=self.device)
        self.prefill_ws = torch.empty(_words(self.prefill_bytes), dtype=torch.int32, device=self.device)
        # An empty visible_lens tells the decode op to derive causal ends from seq_lens.
        self.visible = torch.empty((0,), dtype=torch.int32, device=self.device)
        self._legacy: dict[str, torch.Tensor] = {}

    @property
    def nbytes(self) -> int:
        """Device bytes this scratch holds (the two workspaces)."""
        return 4 * (self.decode_ws.numel() + self.prefill_ws.numel())

    def workspace(self, nprog: int) -> tuple[torch.Tensor, None, None, None]:
        """The decode workspace in the reference's ``(partials, m, l, merged)`` slot order.

        Only the first entry is a buffer: the split states live there, so the
        reference's m / l / merged workspaces are None."""
        if not 1 <= int(nprog) <= self.nprog_max:
            raise RuntimeError(
                "K8/V4 workspace needs %d programs and was allocated for %d" % (int(nprog), self.nprog_max)
            )
        return self.decode_ws, None, None, None

    # -- objects kept for callers written against the reference's scratch ------
    def _lazy(self, name: str, shape: tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
        t = self._legacy.get(name)
        if t is None:
            t = self._legacy[name] = torch.zeros(shape, dtype=dtype, device=self.device)
        return t

    @property
    def q8(self) -> torch.Tensor:
        """The reference's int8 query tile ``[hkv, 64, D]`` (created on first use)."""
        return self._lazy("q8", (self.layout.hkv, PAGE, self.layout.head_dim), torch.int8)

    @property
    def q_scale(self) -> torch.Tensor:
        """The reference's query scales ``[hkv, 64]`` (created on first use)."""
        return self._lazy("q_scale", (self.layout.hkv, PAGE), torch.float32)

    def store_pair(self, ntok: int) -> tuple[torch.Tensor, torch.Tensor]:
        """fp16 key/value rows for ``ntok`` tokens (created on first use; the backend stores in place)."""
        n = int(ntok)
        if not 1 <= n <= self.max_store_tokens:
            raise RuntimeError("K8/V4 store buffer holds %d tokens, got %d" % (self.max_store_tokens, n))
        shape = (self.max_store_tokens, self.layout.hkv, self.layout.head_dim)
        return self._lazy("k16", shape, torch.float16)[:n], self._lazy("v16", shape, torch.float16)[:n]

    def attention_pair(self, ntok: int) -> tuple[torch.Tensor, torch.Tensor]:
        """fp16 query/output rows for ``ntok`` tokens (created on first use; the backend decodes in place)."""
        n = int(ntok)
        if not 1 <= n <= self.max_out_tokens:
            raise RuntimeError("K8/V4 attention buffer holds %d tokens, got %d" % (self.max_out_tokens, n))
        shape = (self.max_out_tokens, self.layout.hq, self.layout.head_dim)
        return self._lazy("q16", shape, torch.float16)[:n], self._lazy("o16", shape, torch.float16)[:n]

    def covers(self, nprog_max: int, max_store_tokens: int, max_out_tokens: int, max_seqs: int | None = None) -> bool:
        seqs_ok = self.max_seqs is None or (max_seqs is not None and self.max_seqs >= int(max_seqs))
        return (self.nprog_max >= int(nprog_max) and self.max_store_tokens >= int(max_store_tokens)
                and self.max_out_tokens >= int(max_out_tokens) and seqs_ok)


def _words(nbytes: int) -> int:
    """int32 elements of a buffer of at least ``nbytes`` (never empty)."""
    return max(4, -(-int(nbytes) // 4))


def scratch_key(device: torch.device, layout: PageLayout) -> tuple[str, int | None, int, int]:
    """Registry key; ``cuda`` and ``cuda:<current>`` name the same device."""
    device = torch.device(device)
    index = device.index
    if index is None and device.type == "cuda":
        index = torch.cuda.current_device()
    return device.type, index, layout.hkv, layout.head_dim


def ensure_scratch(device, layout: PageLayout, nprog_max: int, max_store_tokens: int, max_out_tokens: int,
                   max_seqs: int | None = None) -> Scratch:
    """The registered scratch of (device, layout), replaced by a larger one when it is too small.

    ``max_seqs`` (optional) caps the sequences of one decode call; without it
    the decode workspace covers ``max_out_tokens`` one-token sequences."""
    key = scratch_key(device, layout)
    have = _REGISTRY.get(key)
    if have is None or not have.covers(nprog_max, max_store_tokens, max_out_tokens, max_seqs):
        if have is not None:
            nprog_max = max(int(nprog_max), have.nprog_max)
            max_store_tokens = max(int(max_store_tokens), have.max_store_tokens)
            max_out_tokens = max(int(max_out_tokens), have.max_out_tokens)
            if max_seqs is not None and have.max_seqs is not None:
                max_seqs = max(int(max_seqs), have.max_seqs)
            else:
                max_seqs = None
        have = _REGISTRY[key] = Scratch(device, layout, nprog_max, max_store_tokens, max_out_tokens, max_seqs)
    return have


def get_scratch(device, layout: PageLayout) -> Scratch:
    have = _REGISTRY.get(scratch_key(device, layout))
    if have is None:
        raise RuntimeError("K8/V4 scratch was not allocated before attention")
    return have


def scratch_ready(device, layout: PageLayout) -> bool:
    return scratch_key(device, layout) in _REGISTRY


def clear_scratch() -> None:
    _REGISTRY.clear()


__all__ = ["Scratch", "clear_scratch", "decode_workspace_bytes", "ensure_scratch", "get_scratch",
           "prefill_workspace_bytes", "scratch_key", "scratch_ready"]
