"""vLLM attention backend for the K8/V4 cache on MI355X (2 or 4 local KV heads).

This is the caller of the hot path: vLLM owns the block table and the slot
map; the backend turns one engine step's metadata into the library's three
entry points (quantize-and-write, batched decode / MTP verify, chunked
prefill).  The vLLM-facing surface follows the reference backend
(k8v4_v030/backend.py:56-486): the class names, the metadata fields, the
constructor and forward signatures, the capture support and the error
messages callers and tests match.  The implementation is this package's own:

* the metadata builder turns ``query_start_loc`` into a step plan once per
  step (decode runs of equal query length, and the prefill sequences), which
  every layer's ``forward`` then walks;
* vLLM's fp16/bf16 ``query`` / ``key`` / ``value`` / ``output`` rows go to
  the kernels in place (they take token strides and bf16), so there are no
  staging copies;
* decode runs use the scratch's decode workspace and prefill sequences its
  prefill workspace, both allocated before capture (``scratch.py``), so no
  call allocates;
* a step made only of decode runs of one query length is one launch pair and
  can be captured in a HIP graph; a step with prefill refuses capture.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from vllm.logger import init_logger
from vllm.v1.attention.backend import (
    AttentionBackend,
    AttentionCGSupport,
    AttentionImpl,
    AttentionMetadata,
    AttentionMetadataBuilder,
    AttentionType,
    CommonAttentionMetadata,
    MultipleOf,
)
from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend
from vllm.v1.kv_cache_interface import AttentionSpec

from .cache_views import bind_regions
from .layout import CACHE_DTYPE, DECODE_MAX_T, PAGE, PageLayout, attention_pages_per_block
from .ops_api import ops
from .plan import layout_for_heads, query_segments, require_decoder, scratch_capacity, token_span, uniform_packed_q_len
from .scratch import Scratch, ensure_scratch, get_scratch, scratch_ready

logger = init_logger(__name__)

_REGIONS = ("k", "k_scale", "v", "v_scale", "v_zero")


# --------------------------------------------------------------- step plan
@dataclass(frozen=True)
class DecodeRun:
    """Requests ``first .. first + count - 1``, each with ``q_len`` query tokens
    packed from token ``tok0``: one batched decode launch."""

    first: int
    count: int
    q_len: int
    tok0: int


@dataclass(frozen=True)
class PrefillSeq:
    """Request ``req``'s ``width`` query tokens from token ``tok0``: one prefill launch."""

    req: int
    tok0: int
    width: int


def plan_step(query_starts: tuple[int, ...]) -> tuple[tuple[DecodeRun, ...], tuple[PrefillSeq, ...]]:
    """Split a step into decode runs (1..10 query tokens) and prefill sequences (longer)."""
    runs: list[DecodeRun] = []
    seqs: list[PrefillSeq] = []
    for first, count, q_len in query_segments(query_starts):
        if q_len == 0:
            continue
        if q_len <= DECODE_MAX_T:
            tok0, _ = token_span(query_starts, first, count, q_len)
            runs.append(DecodeRun(first, count, q_len, tok0))
        else:
            for req in range(first, first + count):
                tok0, width = token_span(query_starts, req, 1, q_len)
                seqs.append(PrefillSeq(req, tok0, width))
    return tuple(runs), tuple(seqs)


def attention_pages(manager_block: int, kernel_block: int | None) -> int:
    """Kernel pages per block-table entry (layout.attention_pages_per_block)."""
    return attention_pages_per_block(int(manager_block), kernel_block)


# ---------------------------------------------------------------- metadata
class Xe2K8V4Metadata(AttentionMetadata):
    """One step's attention metadata (fields of backend.py:82-110) plus its plan."""

    def __init__(
        self,
        seq_lens: torch.Tensor,
        slot_mapping: torch.Tensor,
        block_table: torch.Tensor,
        query_start_loc: torch.Tensor,
        query_starts: tuple[int, ...],
        seq_lens_cpu: torch.Tensor | None,
        num_actual_tokens: int,
        max_query_len: int,
        max_seq_len: int,
        pages_per_block: int,
        packed_q_len: int,
        layout: PageLayout,
    ):
        for name, value in list(locals().items()):
            if name != "self":
                setattr(self, name, value)
        self.decode_runs, self.prefill_seqs = plan_step(tuple(query_starts))


class Xe2K8V4MetadataBuilder(AttentionMetadataBuilder[Xe2K8V4Metadata]):
    """Per-step metadata and the device scratch, sized from the engine config.

    A uniform batch (every request 1..10 query tokens, the same count) is one
    decode launch and may be captured; MTP verify steps join the decode group.
    """

    _cudagraph_support = AttentionCGSupport.UNIFORM_BATCH

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        self.layout = PageLayout(int(kv_cache_spec.num_kv_heads), int(getattr(kv_cache_spec, "head_size", 256)))
        logger.info_once("K8/V4 local heads: %d KV / %d Q", self.layout.hkv, self.layout.hq)
        self._init_reorder_batch_threshold(1, supports_spec_as_decode=True)

    def _pages_per_entry(self) -> int:
        return attention_pages(self.kv_cache_spec.block_size, getattr(self, "kernel_block_size", None))

    def set_kernel_block_size(self, kernel_block_size: int) -> None:
        super().set_kernel_block_size(kernel_block_size)
        logger.info_once(
            "K8/V4 pages per block-table entry: %d (manager block %d, kernel block %s)",
            self._pages_per_entry(),
            int(self.kv_cache_spec.block_size),
            self.kernel_block_size,
        )
        self._ensure_scratch()

    def _ensure_scratch(self) -> Scratch:
        cfg = self.vllm_config
        capture = getattr(getattr(cfg, "compilation_config", None), "cudagraph_capture_sizes", None) or []
        capacity = scratch_capacity(
            int(cfg.model_config.max_model_len),
            int(self.kv_cache_spec.block_size),
            getattr(self, "kernel_block_size", None),
            int(cfg.scheduler_config.max_num_batched_tokens),
            int(cfg.scheduler_config.max_num_seqs),
            list(capture),
            self.layout,
        )
        return ensure_scratch(self.device, self.layout, *capacity, max_seqs=int(cfg.scheduler_config.max_num_seqs))

    def build(
        self,
        common_prefix_len: int,
        common_attn_metadata: CommonAttentionMetadata,
        fast_build: bool = False,
    ) -> Xe2K8V4Metadata:
        del common_prefix_len, fast_build
        if not scratch_ready(self.device, self.layout):
            self._ensure_scratch()
        cam = common_attn_metadata
        starts = tuple(int(x) for x in cam.query_start_loc_cpu.tolist())
        return Xe2K8V4Metadata(
            seq_lens=cam.seq_lens,
            slot_mapping=cam.slot_mapping,
            block_table=cam.block_table_tensor,
            query_start_loc=cam.query_start_loc,
            query_starts=starts,
            seq_lens_cpu=cam.seq_lens_cpu_upper_bound,
            num_actual_tokens=int(cam.num_actual_tokens),
            max_query_len=int(cam.max_query_len),
            max_seq_len=int(cam.max_seq_len),
            pages_per_block=self._pages_per_entry(),
            packed_q_len=uniform_packed_q_len(starts),
            layout=self.layout,
        )


# --------------------------------------------------------------- the layer
class Xe2K8V4Impl(AttentionImpl[Xe2K8V4Metadata]):
    """Quantize-and-write and attention of one layer."""

    def __init__(
        self,
        num_heads: int,
        head_size: int,
        scale: float,
        num_kv_heads: int | None = None,
        alibi_slopes: torch.Tensor | None = None,
        sliding_window: int | None = None,
        kv_cache_dtype: str = "auto",
        logits_soft_cap: float | None = None,
        attn_type: str = AttentionType.DECODER,
        kv_sharing_target_layer_name: str | None = None,
        sinks: torch.Tensor | None = None,
    ) -> None:
        # A sink bias is not implemented; refusing it beats dropping it.
        if sinks is not None:
            raise RuntimeError("Xe2K8V4Impl: attention sink bias (sinks) is not implemented on the k8v4 backend")
        if kv_cache_dtype != CACHE_DTYPE:
            raise RuntimeError("K8/V4 impl got kv dtype %s" % kv_cache_dtype)
        kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        self.layout = layout_for_heads(num_heads, kv_heads, head_size)
        require_decoder(attn_type, sliding_window, alibi_slopes, logits_soft_cap, scale, int(head_size))
        self.num_heads, self.num_kv_heads, self.head_size = num_heads, kv_heads, head_size
        self.scale = float(scale)
        self.kv_cache_dtype = kv_cache_dtype
        self.kv_sharing_target_layer_name = kv_sharing_target_layer_name

    # -- store ---------------------------------------------------------------
    def do_kv_cache_update(
        self,
        layer: torch.nn.Module,
        key: torch.Tensor,
        value: torch.Tensor,
        kv_cache: torch.Tensor,
        slot_mapping: torch.Tensor,
    ) -> None:
        del layer
        cache = _cache_tensor(kv_cache)
        if cache.numel() == 0:
            return
        if slot_mapping.ndim != 1:
            raise RuntimeError("slot_mapping rank %d" % slot_mapping.ndim)
        ntok = int(slot_mapping.shape[0])
        if ntok == 0:
            return
        if slot_mapping.dtype != torch.int64 or not slot_mapping.is_contiguous():
            raise RuntimeError("slot_mapping must be contiguous int64, got %s stride %s"
                               % (slot_mapping.dtype, tuple(slot_mapping.stride())))
        if min(int(key.shape[0]), int(value.shape[0])) < ntok:
            raise RuntimeError("key/value shorter than slot_mapping")
        regions = _regions(cache, self.layout)
        k = _rows(key[:ntok], self.layout.hkv, self.layout.head_dim, "key")
        v = _rows(value[:ntok], self.layout.hkv, self.layout.head_dim, "value")
        ops().kv_store_paged(k, v, slot_mapping, *regions)

    # -- attention -----------------------------------------------------------
    def forward(
        self,
        layer: torch.nn.Module,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        kv_cache: torch.Tensor,
        attn_metadata: Xe2K8V4Metadata,
        output: torch.Tensor,
        output_scale: torch.Tensor | None = None,
        output_block_scale: torch.Tensor | None = None,
    ) -> torch.Tensor:
        del layer, key, value
        if output_scale is not None or output_block_scale is not None:
            raise RuntimeError("K8/V4 does not take an output scale")
        cache = _cache_tensor(kv_cache)
        if cache.numel() == 0 or query.shape[0] == 0:
            return output
        meta = attn_metadata
        if meta.layout != self.layout:  # builder (cache spec) and impl (module) disagree
            raise RuntimeError(
                "K8/V4 KV cache was built for %d KV / %d Q heads but the attention impl derived %d KV / %d Q"
                % (meta.layout.hkv, meta.layout.hq, self.layout.hkv, self.layout.hq))
        _check_block_geometry(cache, meta.pages_per_block, self.layout)
        lay = self.layout
        q = _rows(query, lay.hq, lay.head_dim, "query")
        out = _rows(output, lay.hq, lay.head_dim, "output")
        regions = _regions(cache, lay)
        scratch = get_scratch(query.device, lay)
        if meta.packed_q_len:
            runs = meta.decode_runs
            if meta.prefill_seqs or len(runs) != 1 or runs[0].q_len != int(meta.packed_q_len):
                raise RuntimeError("packed metadata does not match query starts")
        elif _graph_capturing():
            raise RuntimeError("K8/V4 prefill cannot run inside a HIP graph")
        for run in meta.decode_runs:
            self._decode(q, out, regions, meta, run, scratch)
        if meta.prefill_seqs:
            lens = meta.seq_lens_cpu if meta.seq_lens_cpu is not None else meta.seq_lens.detach().cpu()
            alone = [_runs_alone(seq.width, int(lens[seq.req]), lay) for seq in meta.prefill_seqs]
            short = [seq for seq, a in zip(meta.prefill_seqs, alone) if not a]
            if short:
                self._prefill_batch(q, out, regions, meta, short, lens, scratch)
            for seq, a in zip(meta.prefill_seqs, alone):
                if a:
                    self._prefill(q, out, regions, meta, seq, int(lens[seq.req]), scratch)
        return output

    def _decode(self, q, out, regions, meta: Xe2K8V4Metadata, run: DecodeRun, scratch: Scratch) -> None:
        width = run.count * run.q_len
        if q.shape[0] < run.tok0 + width:
            raise RuntimeError("query shorter than the packed segment")
        table = meta.block_table
        if table.ndim != 2 or table.shape[0] < run.first + run.count:
            raise RuntimeError("block_table shape %s" % (tuple(table.shape),))
        table = table[run.first : run.first + run.count]
        if table.dtype != torch.int32 or not table.is_contiguous():
            raise RuntimeError("block_table must be contiguous int32, got %s stride %s"
                               % (table.dtype, tuple(table.stride())))
        lens = meta.seq_lens
        if lens.dtype != torch.int32 or not lens.is_contiguous():
            raise RuntimeError("seq_lens must be contiguous int32, got %s stride %s"
                               % (lens.dtype, tuple(lens.stride())))
        lens = lens.reshape(-1)[run.first : run.first + run.count]
        rows = slice(run.tok0, run.tok0 + width)
        ops().int8k_int4v_attn_batch(q[rows], None, None, *regions, table, lens, None, scratch.decode_ws,
                                     None, None, None, out[rows], run.q_len, meta.pages_per_block)

    def _prefill_batch(self, q, out, regions, meta: Xe2K8V4Metadata, seqs: list[PrefillSeq], lens,
                       scratch: Scratch) -> None:
        """The step's short chunks in one call (the reference runs one prefill per
        request, backend.py:376-409)."""
        seq_lens = [int(lens[seq.req]) for seq in seqs]
        for seq, seq_len in zip(seqs, seq_lens):
            _check_covers(seq_len, seq.width)
        table = meta.block_table
        if table.dtype != torch.int32 or table.dim() != 2 or table.stride(1) != 1:
            table = table.to(torch.int32).contiguous()
        ops().prefill_paged_batch(q, *regions, table, [seq.tok0 for seq in seqs], [seq.width for seq in seqs],
                                  seq_lens, [seq.req for seq in seqs], meta.pages_per_block, self.scale, out,
                                  workspace=scratch.prefill_ws)

    def _prefill(self, q, out, regions, meta: Xe2K8V4Metadata, seq: PrefillSeq, seq_len: int,
                 scratch: Scratch) -> None:
        _check_covers(seq_len, seq.width)
        row = meta.block_table[seq.req]
        if row.dtype != torch.int32 or not row.is_contiguous():
            row = row.to(torch.int32).contiguous()
        rows = slice(seq.tok0, seq.tok0 + seq.width)
        ops().prefill_paged(q[rows], *regions, row, seq_len, meta.pages_per_block, self.scale, out[rows],
                            workspace=scratch.prefill_ws)


# ----------------------------------------------------------------- helpers
# Chunks the single prefill entry would run with its in-kernel page conversion
# gain nothing from running alone: a step's share one batched launch.  A chunk
# the single entry serves from per-head tile images (each page dequantized
# once per KV head: at head dim 128 over 128 tokens; at head dim 256 long
# chunks over long contexts) runs alone.  The library's plan decides.
def _runs_alone(width: int, seq_len: int, layout) -> bool:
    _check_covers(seq_len, width)
    return ops().prefill_uses_tiles(seq_len, width, layout.hkv, layout.head_dim)


def _check_covers(seq_len: int, width: int) -> None:
    if seq_len < width:
        raise RuntimeError("seq_len %d does not cover query %d; the kernel expects the length to include "
                           "this step" % (seq_len, width))

def _cache_tensor(kv_cache) -> torch.Tensor:
    """The layer's one packed cache tensor (vLLM may hand it over in a list)."""
    if isinstance(kv_cache, (list, tuple)):
        if len(kv_cache) != 1:
            raise RuntimeError("K8/V4 cache is one packed tensor, got %d pieces" % len(kv_cache))
        kv_cache = kv_cache[0]
    return kv_cache


def _check_block_geometry(cache: torch.Tensor, pages_per_block: int, layout: PageLayout) -> None:
    """The cache is ``[block, head, token, slot_bytes]`` and one block is ``pages_per_block`` pages.

    (The reference's page-ratio rule, backend.py:59-79; a 2,112-token manager
    block is 33 kernel pages and goes to the kernels as such.)"""
    slot = layout.slot_bytes_per_head
    if cache.ndim != 4 or int(cache.shape[-1]) != slot:
        raise RuntimeError("K8/V4 cache shape %s is not [block, head, token, %d]" % (tuple(cache.shape), slot))
    tokens = int(cache.shape[-2])
    if tokens % PAGE:
        raise RuntimeError("K8/V4 block has %d tokens, not a multiple of %d" % (tokens, PAGE))
    if tokens // PAGE != int(pages_per_block):
        raise RuntimeError("K8/V4 pages_per_block %s does not match the %d-token cache block (%d pages)"
                           % (pages_per_block, tokens, tokens // PAGE))


def _regions(cache: torch.Tensor, layout: PageLayout) -> tuple[torch.Tensor, ...]:
    views = bind_regions(cache, layout)
    return tuple(views[name] for name in _REGIONS)


def _rows(x: torch.Tensor, heads: int, head_dim: int, what: str) -> torch.Tensor:
    """``[T, heads, D]`` view of vLLM's ``[T, heads * D]`` (or already 3-D) rows, no copy."""
    if x.dim() == 3:
        return x
    if x.dim() == 2 and int(x.shape[1]) == heads * head_dim and x.stride(1) == 1:
        return x.unflatten(1, (heads, head_dim))
    raise RuntimeError("%s shape %s is not [T, %d, %d]" % (what, tuple(x.shape), heads, head_dim))


def _graph_capturing() -> bool:
    return torch.cuda.is_available() and bool(torch.cuda.is_current_stream_capturing())


# ----------------------------------------------------------------- backend
@register_backend(AttentionBackendEnum.CUSTOM)
class Xe2K8V4AttentionBackend(AttentionBackend):
    """The class vLLM's selector returns (registered as the CUSTOM backend)."""

    accept_output_buffer: bool = True
    forward_includes_kv_cache_update: bool = False
    supported_kv_cache_dtypes = [CACHE_DTYPE]

    @staticmethod
    def get_name() -> str:
        # vLLM looks the name up in AttentionBackendEnum; CUSTOM is the
        # member registered for out-of-tree backends.
        return AttentionBackendEnum.CUSTOM.name

    @staticmethod
    def get_impl_cls() -> type[Xe2K8V4Impl]:
        return Xe2K8V4Impl

    @staticmethod
    def get_builder_cls() -> type[Xe2K8V4MetadataBuilder]:
        return Xe2K8V4MetadataBuilder

    @staticmethod
    def get_supported_kernel_block_sizes() -> list[MultipleOf]:
        return [MultipleOf(PAGE)]

    @classmethod
    def get_supported_head_sizes(cls) -> list[int]:
        return [128, 256]

    @classmethod
    def supports_kv_cache_dtype(cls, kv_cache_dtype: str | None) -> bool:
        return kv_cache_dtype == CACHE_DTYPE

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type == AttentionType.DECODER

    @classmethod
    def customize_spec(cls, spec: AttentionSpec) -> AttentionSpec:
        # One (token, KV head) slot: D int8 K, D/2 packed V, three fp32 planes.
        return replace(spec, state_content_bytes=PageLayout(4, int(getattr(spec, "head_size", 256))).slot_bytes_per_head)


__all__ = [
    "DecodeRun",
    "PrefillSeq",
    "Xe2K8V4AttentionBackend",
    "Xe2K8V4Impl",
    "Xe2K8V4Metadata",
    "Xe2K8V4MetadataBuilder",
    "attention_pages",
    "plan_step",
]
