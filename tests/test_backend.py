"""vLLM backend glue on the CPU: registration, spec, rejections and metadata.

Mirrors the checks of the reference's backend (k8v4_v030/backend.py:59-79,
:113-185, :192-270, :446-486) against the stand-in vLLM interface.
"""
from __future__ import annotations

import math

import pytest
import torch

from backend_cases import AttentionType, backend, common_metadata, make_builder, make_impl, vllm_cache
from k8v4_v030.layout import CACHE_DTYPE, PageLayout
from vllm.v1.attention.backend import AttentionCGSupport, MultipleOf
from vllm.v1.attention.backends.registry import REGISTRY, AttentionBackendEnum
from vllm.v1.kv_cache_interface import AttentionSpec


def test_registered_as_the_custom_backend():
    cls = REGISTRY[AttentionBackendEnum.CUSTOM]
    assert cls is backend.Xe2K8V4AttentionBackend
    assert cls.get_name() == "CUSTOM"
    assert AttentionBackendEnum[cls.get_name()] is AttentionBackendEnum.CUSTOM
    assert cls.get_impl_cls() is backend.Xe2K8V4Impl
    assert cls.get_builder_cls() is backend.Xe2K8V4MetadataBuilder
    assert cls.accept_output_buffer and not cls.forward_includes_kv_cache_update
    assert cls.get_supported_kernel_block_sizes() == [MultipleOf(64)]
    assert cls.supports_kv_cache_dtype(CACHE_DTYPE) and not cls.supports_kv_cache_dtype("auto")
    assert cls.supports_attn_type(AttentionType.DECODER) and not cls.supports_attn_type(AttentionType.ENCODER)
    assert backend.Xe2K8V4MetadataBuilder._cudagraph_support is AttentionCGSupport.UNIFORM_BATCH


@pytest.mark.parametrize("head,slot", [(128, 204), (256, 396)])
def test_spec_carries_the_slot_bytes(head, slot):
    spec = AttentionSpec(block_size=64, num_kv_heads=4, head_size=head)
    assert backend.Xe2K8V4AttentionBackend.customize_spec(spec).state_content_bytes == slot
    assert PageLayout(4, head).slot_bytes_per_head == slot


def test_impl_rejections():
    make_impl()  # the supported configuration
    with pytest.raises(RuntimeError, match="attention sink bias"):
        make_impl(sinks=torch.zeros(24))
    with pytest.raises(RuntimeError, match="K8/V4 impl got kv dtype auto"):
        make_impl(kv_cache_dtype="auto")
    with pytest.raises(RuntimeError, match="12/2 \\(TP2\\) or 24/4"):
        make_impl(num_heads=18, num_kv_heads=3)
    with pytest.raises(RuntimeError, match="head dim"):
        make_impl(head_size=64, scale=1 / 8)
    with pytest.raises(RuntimeError, match="scale is fixed"):
        make_impl(scale=0.1)
    with pytest.raises(RuntimeError, match="sliding window"):
        make_impl(sliding_window=128)
    with pytest.raises(RuntimeError, match="alibi"):
        make_impl(alibi_slopes=torch.ones(24))
    with pytest.raises(RuntimeError, match="soft cap"):
        make_impl(logits_soft_cap=30.0)
    with pytest.raises(RuntimeError, match="decoder-only"):
        make_impl(attn_type=AttentionType.ENCODER)
    impl = make_impl(hkv=2, head=256)
    assert impl.layout == PageLayout(2, 256) and impl.scale == pytest.approx(1 / 16)


def test_builder_metadata_and_page_ratio():
    b = make_builder(block_size=2112, kernel_block=None)
    table = torch.zeros((3, 2), dtype=torch.int32)
    meta = b.build(0, common_metadata([7, 7, 7], [100, 2000, 3000], table, torch.zeros(21, dtype=torch.int64),
                                      "cpu"))
    assert meta.packed_q_len == 7 and meta.pages_per_block == 33 and meta.query_starts == (0, 7, 14, 21)
    assert meta.layout == PageLayout(4, 128) and meta.max_query_len == 7 and meta.num_actual_tokens == 21
    mixed = b.build(0, common_metadata([1, 1, 50], [10, 20, 50], table, torch.zeros(52, dtype=torch.int64), "cpu"))
    assert mixed.packed_q_len == 0
    b64 = make_builder(block_size=2112, kernel_block=64)
    assert b64.build(0, common_metadata([1], [5], table[:1], torch.zeros(1, dtype=torch.int64),
                                        "cpu")).pages_per_block == 1


def test_page_ratio_and_shape_checks():
    lay = PageLayout(4, 128)
    cache = vllm_cache(2, 128, lay, "cpu")
    backend._check_block_geometry(cache, 2, lay)
    with pytest.raises(RuntimeError, match="pages_per_block 1 does not match the 128-token cache block"):
        backend._check_block_geometry(cache, 1, lay)
    with pytest.raises(RuntimeError, match="is not \\[block, head, token, 204\\]"):
        backend._check_block_geometry(cache.view(2, 4, 128 * 204), 2, lay)
    with pytest.raises(RuntimeError, match="one packed tensor"):
        backend._cache_tensor([cache, cache])
    assert backend._cache_tensor((cache,)) is cache


def test_step_plan_splits_decode_runs_and_prefill_sequences():
    """The builder plans a step once: runs of 1..10 query tokens are batched
    decode launches, longer queries one prefill launch per sequence."""
    runs, seqs = backend.plan_step((0, 7, 14, 21))
    assert runs == (backend.DecodeRun(0, 3, 7, 0),) and seqs == ()
    # decode q=1 x2, a 50-token prefill, decode q=1, an empty request, two 12-token prefills
    starts = (0, 1, 2, 52, 53, 53, 65, 77)
    runs, seqs = backend.plan_step(starts)
    assert runs == (backend.DecodeRun(0, 2, 1, 0), backend.DecodeRun(3, 1, 1, 52))
    assert seqs == (backend.PrefillSeq(2, 2, 50), backend.PrefillSeq(5, 53, 12), backend.PrefillSeq(6, 65, 12))
    b = make_builder()
    table = torch.zeros((7, 4), dtype=torch.int32)
    meta = b.build(0, common_metadata([1, 1, 50, 1, 0, 12, 12], [10, 20, 60, 30, 5, 100, 100], table,
                                      torch.zeros(77, dtype=torch.int64), "cpu"))
    assert meta.decode_runs == runs and meta.prefill_seqs == seqs and meta.packed_q_len == 0


def test_forward_refuses_output_scale_and_layout_mismatch():
    impl = make_impl()
    lay = PageLayout(4, 128)
    cache = vllm_cache(1, 64, lay, "cpu")
    b = make_builder(hkv=2)
    meta = b.build(0, common_metadata([1], [1], torch.zeros((1, 1), dtype=torch.int32),
                                      torch.zeros(1, dtype=torch.int64), "cpu"))
    q = torch.zeros((1, 24, 128), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="output scale"):
        impl.forward(None, q, None, None, cache, meta, torch.empty_like(q), output_scale=torch.ones(1))
    with pytest.raises(RuntimeError, match="built for 2 KV / 12 Q heads but the attention impl derived 4 KV / 24 Q"):
        impl.forward(None, q, None, None, cache, meta, torch.empty_like(q))
    # Empty inputs return the output untouched (no library call).
    out = torch.full((0, 24, 128), 1.0, dtype=torch.float16)
    assert impl.forward(None, q[:0], None, None, cache, meta, out) is out


def test_store_argument_checks():
    impl = make_impl()
    cache = vllm_cache(1, 64, PageLayout(4, 128), "cpu")
    k = torch.zeros((4, 4, 128), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="slot_mapping rank 2"):
        impl.do_kv_cache_update(None, k, k, cache, torch.zeros((2, 2), dtype=torch.int64))
    with pytest.raises(RuntimeError, match="slot_mapping must be contiguous int64"):
        impl.do_kv_cache_update(None, k, k, cache, torch.zeros(4, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="key/value shorter than slot_mapping"):
        impl.do_kv_cache_update(None, k, k, cache, torch.zeros(5, dtype=torch.int64))
    impl.do_kv_cache_update(None, k, k, cache, torch.zeros(0, dtype=torch.int64))  # nothing to store


def test_heads_views_of_vllm_rows():
    qkv = torch.zeros((3, (24 + 8) * 128))
    q = qkv[:, : 24 * 128]
    v = backend._rows(q, 24, 128, "query")
    assert v.shape == (3, 24, 128) and v.data_ptr() == q.data_ptr() and v.stride(0) == 32 * 128
    k = backend._rows(qkv[:, 24 * 128 : 28 * 128], 4, 128, "key")
    assert k.shape == (3, 4, 128) and k.stride() == (32 * 128, 128, 1)
    with pytest.raises(RuntimeError, match="is not \\[T, 24, 128\\]"):
        backend._rows(torch.zeros((3, 100)), 24, 128, "query")
    assert math.isclose(backend.attention_pages(2112, None), 33)


def _words_bytes(n: int) -> int:
    return 4 * (-(-int(n) // 4))


@pytest.mark.parametrize("hkv,head,max_model_len,max_seqs,max_batched",
                         [(4, 128, 4096, 256, 8192), (2, 256, 4096, 256, 8192), (4, 128, 131072, 8, 8192),
                          (2, 256, 200000, 64, 16384)])
def test_scratch_covers_every_decode_call_the_engine_can_issue(hkv, head, max_model_len, max_seqs, max_batched):
    """The decode workspace is sized by the library for the widest call of
    every query length (a batch of short sequences needs more split states
    than the reference's pages x heads sizing gave it), and the scratch holds
    only the two workspaces the kernels use."""
    from k8v4_v030.ops_api import ops
    from k8v4_v030.scratch import clear_scratch, get_scratch

    clear_scratch()
    b = make_builder(hkv=hkv, head=head, max_model_len=max_model_len, max_seqs=max_seqs,
                     max_batched=max_batched, capture=(1, 2, 4, 8, 16))
    s = get_scratch(torch.device("cpu"), b.layout)
    lib = ops()
    pages = -(-max_model_len // 64) + 1
    max_out = max(max_seqs * 10, 16)
    sized = 0
    for q_len in range(1, 11):
        batch = max_seqs
        need = lib.attn_workspace_bytes(batch, pages, 1, q_len, hkv, head)
        assert s.decode_ws.numel() * 4 >= need, (q_len, need)
        sized = max(sized, lib.attn_workspace_bytes(min(max_seqs, max_out // q_len), pages, 1, q_len, hkv, head))
    # No larger than that: a call never holds more sequences than the engine schedules.
    assert s.decode_bytes == sized and s.max_seqs == max_seqs
    assert s.prefill_ws.numel() * 4 >= lib.prefill_workspace_bytes(min(max_batched, pages * 64), min(max_batched, pages * 64), hkv, head)
    # Nothing besides the two workspaces; less than the reference's
    # [pages x heads, 64, D] fp32 partials once contexts are long (the prefill
    # workspace grows with one head's tile images: 200,000 tokens at D = 256
    # take about 217 MB of them).
    assert s.nbytes == _words_bytes(s.decode_bytes) + _words_bytes(s.prefill_bytes)
    if max_model_len >= 131072:
        assert s.nbytes < pages * hkv * 64 * head * 4
    ws, m, l, merged = s.workspace(1)
    assert ws is s.decode_ws and m is None and l is None and merged is None
    assert s.q8.shape == (hkv, 64, head) and s.q_scale.shape == (hkv, 64)  # created on first use
    clear_scratch()


def test_prefill_plan_query_reports_a_short_sequence_length():
    """A prefill whose sequence length does not include its own query tokens
    is refused with the length message before any prefill launch is planned."""
    lay = PageLayout(hkv=4, head_dim=128)
    with pytest.raises(RuntimeError, match="seq_len 5 does not cover query 10"):
        backend._runs_alone(10, 5, lay)
    assert backend._runs_alone(4, 100, lay) is False
    assert backend._runs_alone(2048, 4096, lay) is True
