"""ctypes boundary into the gfx950 HIP library (``libk8v4_hip.so``).

``ops()`` returns an object whose methods carry the names and argument orders
of the reference's ``torch.ops.xe2_kv`` ops (k8v4_v030/ops_api.py:14-25,
native/xe2_kv_ops.cpp:1779-1822), so callers written against the reference
keep working.  Each method validates its tensors the way the reference's
``TORCH_CHECK``s do (dtypes, ranks, within-page strides, the 2-or-4 head
rule, with the same messages) and then passes raw device pointers, sizes and
the current HIP stream to the C ABI declared in ``include/k8v4_abi.h``.
Errors come back as ``RuntimeError``.  There is no fallback: a missing
library raises ``FileNotFoundError`` and a CPU tensor raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

from .layout import GQA, PAGE

_DEFAULT_LIB = Path(__file__).resolve().parent / "libk8v4_hip.so"
_LIB = None
_LOADED: str | None = None
_OPS = None

F16, BF16, F32 = 0, 1, 2
_DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_vp = ctypes.c_void_p


def library_path() -> str:
    """``K8V4_HIP_LIB`` if set, else the in-tree build."""
    return os.environ.get("K8V4_HIP_LIB", str(_DEFAULT_LIB))


def _declare(lib: ctypes.CDLL) -> None:
    lib.k8v4_abi_version.restype = _i32
    lib.k8v4_abi_version.argtypes = []
    lib.k8v4_last_error.restype = ctypes.c_char_p
    lib.k8v4_last_error.argtypes = []
    lib.k8v4_kv_store_paged.restype = _i32
    lib.k8v4_kv_store_paged.argtypes = [
        _vp, _vp, _i32, _i64, _i64, _vp, _i64, _i32, _i32,
        _vp, _vp, _vp, _vp, _vp,
        _i64, _i64, _i64, _i64, _i64, _i64, _vp,
    ]
    for name, argtypes, restype in _EXTRA_SYMBOLS:
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype


# Entry points beyond the store: (name, argtypes, restype).
_EXTRA_SYMBOLS: list[tuple[str, list, object]] = [
    (
        "k8v4_attn_batch",
        [_vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp, _i64, _i64, _i32, _vp, _vp, _i64, _i64, _i32, _i32, _i32,
         _vp, _i32, _i64, _vp, _i64, _i32, _vp],
        _i32,
    ),
    ("k8v4_attn_workspace_bytes", [_i64, _i64, _i32, _i32, _i32, _i32, _i32], _i64),
]
_EXTRA_SYMBOLS.append(("k8v4_attn_batch_profiled", _EXTRA_SYMBOLS[0][1] + [_vp, _i32], _i32))
_EXTRA_SYMBOLS.append((
    "k8v4_prefill_paged",
    [_vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
     _vp, _i64, _i32, _i64, _i64, _i32, _i32, ctypes.c_float, _vp, _i32, _i64, _vp, _i64, _vp],
    _i32,
))
_EXTRA_SYMBOLS.append(("k8v4_prefill_workspace_bytes", [_i64, _i64, _i32, _i32], _i64))
_EXTRA_SYMBOLS.append(("k8v4_prefill_uses_tiles", [_i64, _i64, _i32, _i32], _i32))
_EXTRA_SYMBOLS.append((
    "k8v4_prefill_paged_batch",
    [_vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
     _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, _vp, _i32, _i64, _vp, _i64, _vp],
    _i32,
))
_EXTRA_SYMBOLS.append(("k8v4_prefill_batch_workspace_bytes", [_i32, _i32], _i64))
_EXTRA_SYMBOLS.append(("k8v4_k_store_paged", [_vp, _i32, _i64, _vp, _i64, _i32, _i32, _vp, _vp, _i64, _i64, _i64, _vp],
                       _i32))
_EXTRA_SYMBOLS.append(("k8v4_v_store_paged",
                       [_vp, _i32, _i64, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp], _i32))
_EXTRA_SYMBOLS.append(("k8v4_q_quant", [_vp, _i32, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp], _i32))
_EXTRA_SYMBOLS.append((
    "k8v4_attn_batch_q8",
    [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
     _vp, _i64, _i64, _i32, _vp, _vp, _i64, _i64, _i32, _i32, _i32,
     _vp, _i32, _i64, _vp, _i64, _i32, _vp],
    _i32,
))
_EXTRA_SYMBOLS.append(("k8v4_attn_batch_noalloc", _EXTRA_SYMBOLS[0][1][:28] + [_i32, _vp], _i32))
_EXTRA_SYMBOLS.append(("k8v4_attn_noalloc_max_bytes", [], _i64))
_EXTRA_SYMBOLS.append(("k8v4_decode_fault_count", [], _i64))
Q_TOKENS, Q_PADDED = 0, 1


def load_library():
    """Load the shared library once per process (path from :func:`library_path`)."""
    global _LIB, _LOADED
    path = library_path()
    if _LOADED != path:
        if not os.path.isfile(path):
            raise FileNotFoundError("K8/V4 library is not at %s" % path)
        lib = ctypes.CDLL(path)
        _declare(lib)
        _LIB, _LOADED = lib, path
    return _LIB


def _check(rc: int, lib) -> None:
    if rc != 0:
        raise RuntimeError(lib.k8v4_last_error().decode("utf-8", "replace"))


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _checked_hkv(hkv: int) -> int:
    _require(hkv in (2, 4), "unsupported per-GPU KV head count %d (this library serves 2 or 4)" % hkv)
    return hkv


def _on_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        _require(t.is_cuda, "K8/V4 ops need GPU tensors, got a %s tensor" % t.device.type)
        _require(t.device == dev, "K8/V4 op tensors are on different devices")
    return dev


def _stream(dev: torch.device) -> int:
    return int(torch.cuda.current_stream(dev).cuda_stream)


def _ptr(t: torch.Tensor) -> int:
    return int(t.data_ptr())


def check_paged_k(k_cache: torch.Tensor, k_scale: torch.Tensor, hkv: int, head_dim: int) -> None:
    """Shape and within-page stride rules of the K views (xe2_kv_ops.cpp:1333-1349)."""
    _require(k_cache.dtype == torch.int8, "k_cache int8")
    _require(k_scale.dtype == torch.float32, "k_scale float32")
    _require(
        k_cache.dim() == 4 and tuple(k_cache.shape[1:]) == (PAGE, hkv, head_dim),
        "k_cache [num_blocks,64,%d,%d] NHD" % (hkv, head_dim),
    )
    _require(
        k_scale.dim() == 3 and tuple(k_scale.shape) == (k_cache.shape[0], PAGE, hkv),
        "k_scale [num_blocks,64,%d]" % hkv,
    )
    _require(k_cache.stride()[1:] == (hkv * head_dim, head_dim, 1), "k_cache within-page strides")
    _require(k_scale.stride()[1:] == (hkv, 1), "k_scale within-page strides")


def check_paged_v(v_cache, v_scale, v_zero, hkv: int, head_dim: int) -> None:
    """Shape and within-page stride rules of the V views (xe2_kv_ops.cpp:1352-1370)."""
    cols = head_dim // 2
    _require(v_cache.dtype == torch.uint8, "v_cache uint8 packed int4")
    _require(v_scale.dtype == torch.float32 and v_zero.dtype == torch.float32, "v scale/zero float32")
    _require(
        v_cache.dim() == 4 and tuple(v_cache.shape[1:]) == (PAGE, hkv, cols),
        "v_cache [num_blocks,64,%d,%d] NHD packed" % (hkv, cols),
    )
    _require(v_scale.shape == v_zero.shape, "v_scale/v_zero shape")
    _require(
        v_scale.dim() == 3 and tuple(v_scale.shape) == (v_cache.shape[0], PAGE, hkv),
        "v_scale [num_blocks,64,%d]" % hkv,
    )
    _require(v_cache.stride()[1:] == (hkv * cols, cols, 1), "v_cache within-page strides")
    _require(v_scale.stride()[1:] == (hkv, 1), "v_scale within-page")
    _require(v_zero.stride()[1:] == (hkv, 1), "v_zero within-page")


def cache_args(k_cache, k_scale, v_cache, v_scale, v_zero) -> list[int]:
    """Pointers and byte page strides of the five region views, in ABI order."""
    return [
        _ptr(k_cache), _ptr(k_scale), _ptr(v_cache), _ptr(v_scale), _ptr(v_zero),
        int(k_cache.shape[0]),
        int(k_cache.stride(0)),
        int(k_scale.stride(0)) * 4,
        int(v_cache.stride(0)),
        int(v_scale.stride(0)) * 4,
        int(v_zero.stride(0)) * 4,
    ]


def _src_rows(t: torch.Tensor, name: str, hkv: int, head_dim: int) -> int:
    """Validate a ``[T, hkv, D]`` 16-bit source; returns its token stride in elements."""
    _require(t.dtype in (torch.float16, torch.bfloat16), "%s must be float16 or bfloat16" % name)
    _require(t.dim() == 3 and t.shape[2] == head_dim, "%s [T,HKV,%d]" % (name, head_dim))
    _require(t.shape[1] == hkv, "%s heads" % name)
    _require(t.stride(2) == 1 and t.stride(1) == head_dim, "%s head/dim strides must be (%d, 1)" % (name, head_dim))
    return int(t.stride(0)) if t.shape[0] > 1 else hkv * head_dim


class BoundCall:
    """One validated op call: the C entry point plus its argument list.

    Calling it enqueues the op on the current stream of the call's device;
    the tensors it was bound with are kept alive with it.
    """

    __slots__ = ("_lib", "_fn", "_profiled", "_args", "_dev", "_keep")

    def __init__(self, lib, fn, args, dev, keep, profiled=None):
        self._lib, self._fn, self._profiled = lib, fn, profiled
        self._args, self._dev, self._keep = tuple(args), dev, keep

    def __call__(self, split_done_event=None, stages: int = 3) -> None:
        stream = _stream(self._dev)
        if split_done_event is None and stages == 3:
            rc = self._fn(*self._args, stream)
        else:
            _require(self._profiled is not None, "this op has no staged variant")
            rc = self._profiled(*self._args, stream, int(split_done_event or 0), int(stages))
        _check(rc, self._lib)


class _Ops:
    """Methods named after the reference's ``torch.ops.xe2_kv`` schemas."""

    def __init__(self, lib):
        self._lib = lib
        self._legacy_ws: dict[torch.device, torch.Tensor] = {}

    # -- quantize-and-write ------------------------------------------------
    def kv_store_paged(self, k_fp16, v_fp16, slot_mapping, k_cache, k_scale, v_cache, v_scale, v_zero):
        """Quantize K/V ``[T, HKV, D]`` into the paged cache at ``slot_mapping`` (int64 ``[T]``)."""
        bound = self.bind_kv_store_paged(k_fp16, v_fp16, slot_mapping, k_cache, k_scale, v_cache, v_scale, v_zero)
        if bound is not None:
            bound()

    def bind_kv_store_paged(self, k_fp16, v_fp16, slot_mapping, k_cache, k_scale, v_cache, v_scale, v_zero):
        """Validate a store once; returns a :class:`BoundCall` (None when there are no tokens)."""
        _require(k_fp16.dim() == 3, "k_fp16 [T,HKV,D]")
        head_dim = int(k_fp16.shape[2])
        _require(head_dim in (128, 256), "k_fp16 [T,HKV,D] with D in (128, 256)")
        _require(k_fp16.dtype == v_fp16.dtype, "k/v_fp16 dtypes differ")
        _require(v_fp16.shape == k_fp16.shape, "v_fp16 must match k_fp16")
        _require(slot_mapping.dtype == torch.int64, "slot_mapping int64")
        _require(slot_mapping.is_contiguous(), "slot_mapping must be contiguous")
        hkv = _checked_hkv(int(k_fp16.shape[1]))
        check_paged_k(k_cache, k_scale, hkv, head_dim)
        check_paged_v(v_cache, v_scale, v_zero, hkv, head_dim)
        _require(k_cache.shape[0] == v_cache.shape[0], "k/v num_blocks")
        _require(slot_mapping.numel() == k_fp16.shape[0], "slot_mapping [T]")
        ks = _src_rows(k_fp16, "k_fp16", hkv, head_dim)
        vs = _src_rows(v_fp16, "v_fp16", hkv, head_dim)
        ntok = int(k_fp16.shape[0])
        if ntok == 0:
            return None
        tensors = (k_fp16, v_fp16, slot_mapping, k_cache, k_scale, v_cache, v_scale, v_zero)
        dev = _on_gpu(*tensors)
        args = [
            _ptr(k_fp16), _ptr(v_fp16), _DTYPE_CODE[k_fp16.dtype], ks, vs,
            _ptr(slot_mapping), ntok, hkv, head_dim,
            *cache_args(k_cache, k_scale, v_cache, v_scale, v_zero),
        ]
        return BoundCall(self._lib, self._lib.k8v4_kv_store_paged, args, dev, tensors)

    # -- decode / MTP verify ----------------------------------------------
    def attn_workspace_bytes(self, batch: int, table_width: int, pages_per_block: int, q_len: int,
                             hkv: int, head_dim: int, num_splits: int = 0) -> int:
        """Scratch bytes :meth:`int8k_int4v_attn_batch` needs for this shape."""
        n = int(self._lib.k8v4_attn_workspace_bytes(batch, table_width, pages_per_block, q_len, hkv,
                                                    head_dim, num_splits))
        _require(n > 0, "bad shape for the decode workspace")
        return n

    def int8k_int4v_attn_batch(self, q_fp16, q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero,
                               block_table, seq_lens, visible_lens, partials_ws, m_ws, l_ws, merged_ws,
                               out, q_len, pages_per_block, num_splits: int = 0, split_done_event=None,
                               stages: int = 3):
        """One uniform-q_len decode batch (argument order of the reference op).

        Validates and launches; :meth:`bind_int8k_int4v_attn_batch` takes the
        same arguments and returns the validated call for repeated launches.

        ``q8``, ``q_scale``, ``m_ws``, ``l_ws`` and ``merged_ws`` are accepted for
        signature compatibility and left untouched: Q is quantized inside the
        kernel and the split-K state lives in the bytes of ``partials_ws``.
        ``visible_lens`` is None, an empty tensor (derive causal ends from
        ``seq_lens``) or int32 ``[B, >= 1 + q_len]``.

        Timing hooks (no effect on results): ``split_done_event`` is a raw
        hipEvent_t handle recorded after the split-K kernel; ``stages`` = 1 runs
        only the split-K kernel, 2 only the merge (over the workspace a
        ``stages=1`` call with the same arguments filled), 3 both.
        """
        self.bind_int8k_int4v_attn_batch(
            q_fp16, q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero, block_table, seq_lens,
            visible_lens, partials_ws, m_ws, l_ws, merged_ws, out, q_len, pages_per_block, num_splits,
        )(split_done_event=split_done_event, stages=stages)

    def bind_int8k_int4v_attn_batch(self, q_fp16, q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero,
                                    block_table, seq_lens, visible_lens, partials_ws, m_ws, l_ws, merged_ws,
                                    out, q_len, pages_per_block, num_splits: int = 0):
        """Validate one decode call; returns a :class:`BoundCall` that launches it.

        The call keeps the tensors' device addresses: their contents may change
        between launches (new queries, lengths, tables), their storage may not.
        """
        del q8, q_scale, m_ws, l_ws, merged_ws
        q_len = int(q_len)
        pages_per_block = int(pages_per_block)
        _require(pages_per_block >= 1, "pages_per_block")
        _require(q_len > 0 and q_len * GQA <= PAGE, "q_len*GQA exceeds BM")
        _require(q_fp16.dim() == 3, "q_fp16 [T,HQ,D]")
        head_dim = int(q_fp16.shape[2])
        _require(head_dim in (128, 256), "q_fp16 [T,HQ,D] with D in (128, 256)")
        _require(q_fp16.shape[1] % GQA == 0, "q_fp16 heads must be a multiple of GQA=6")
        hkv = _checked_hkv(int(q_fp16.shape[1]) // GQA)
        _require(q_fp16.dtype in (torch.float16, torch.bfloat16), "q_fp16 must be float16 or bfloat16")
        _require(q_fp16.stride(2) == 1 and q_fp16.stride(1) == head_dim, "q_fp16 head/dim strides")
        _require(out.shape == q_fp16.shape, "out shape")
        _require(out.dtype in (torch.float16, torch.bfloat16, torch.float32), "out float16, bfloat16 or float32")
        _require(out.stride(2) == 1 and out.stride(1) == head_dim, "out head/dim strides")
        _require(q_fp16.shape[0] % q_len == 0, "T must be B*q_len")
        batch = int(q_fp16.shape[0]) // q_len
        _require(batch >= 1, "empty batch")
        check_paged_k(k_cache, k_scale, hkv, head_dim)
        check_paged_v(v_cache, v_scale, v_zero, hkv, head_dim)
        _require(k_cache.shape[0] == v_cache.shape[0], "k/v num_blocks")
        _require(block_table.dtype == torch.int32, "block_table int32")
        _require(block_table.dim() == 2 and block_table.shape[0] == batch, "block_table [B, splits]")
        _require(block_table.stride(1) == 1, "block_table rows must be contiguous")
        _require(int(block_table.shape[1]) > 0, "block_table n_splits")
        _require(seq_lens.dtype == torch.int32 and seq_lens.numel() >= batch, "seq_lens [B]")
        _require(seq_lens.is_contiguous(), "seq_lens XPU contig (graph input)")
        vis_ptr, vis_stride = 0, 0
        if visible_lens is not None and visible_lens.numel() > 0:
            _require(visible_lens.dtype == torch.int32, "visible_lens int32")
            _require(visible_lens.dim() == 2 and visible_lens.shape[0] == batch
                     and visible_lens.shape[1] >= q_len + 1, "visible_lens [B, 1+q_len]")
            _require(visible_lens.stride(1) == 1, "visible_lens rows must be contiguous")
            vis_ptr, vis_stride = _ptr(visible_lens), int(visible_lens.stride(0))
        _require(partials_ws is not None and partials_ws.is_contiguous(), "partials_ws must be a contiguous buffer")
        tensors = (q_fp16, k_cache, k_scale, v_cache, v_scale, v_zero, block_table, seq_lens, out, partials_ws)
        dev = _on_gpu(*tensors)
        ws_bytes = int(partials_ws.numel()) * partials_ws.element_size()
        args = [
            _ptr(q_fp16), _DTYPE_CODE[q_fp16.dtype], int(q_fp16.stride(0)),
            *cache_args(k_cache, k_scale, v_cache, v_scale, v_zero),
            _ptr(block_table), int(block_table.stride(0)), int(block_table.shape[1]), pages_per_block,
            _ptr(seq_lens), vis_ptr, vis_stride, batch, q_len, hkv, head_dim,
            _ptr(out), _DTYPE_CODE[out.dtype], int(out.stride(0)),
            _ptr(partials_ws), ws_bytes, int(num_splits),
        ]
        keep = tensors + ((visible_lens,) if vis_ptr else ())
        return BoundCall(self._lib, self._lib.k8v4_attn_batch, args, dev, keep,
                         profiled=self._lib.k8v4_attn_batch_profiled)

    # -- chunked prefill ----------------------------------------------------
    def prefill_workspace_bytes(self, seq_len: int, q_len: int, hkv: int, head_dim: int) -> int:
        """Scratch bytes :meth:`prefill_paged` needs for this shape."""
        n = int(self._lib.k8v4_prefill_workspace_bytes(int(seq_len), int(q_len), int(hkv), int(head_dim)))
        _require(n >= 0, "bad shape for the prefill workspace")
        return n

    def prefill_uses_tiles(self, seq_len: int, q_len: int, hkv: int, head_dim: int) -> bool:
        """Whether :meth:`prefill_paged` serves this shape from per-KV-head tile
        images (each page dequantized once per head) rather than converting
        pages in place as :meth:`prefill_paged_batch` does."""
        n = int(self._lib.k8v4_prefill_uses_tiles(int(seq_len), int(q_len), int(hkv), int(head_dim)))
        _require(n >= 0, "bad shape for the prefill plan")
        return n == 1

    def prefill_paged(self, q, k_cache, k_scale, v_cache, v_scale, v_zero, block_row, seq_len: int,
                      pages_per_block: int, scale: float, out, workspace=None):
        """Bottom-right causal attention of ``q [q_len, HQ, D]`` over one sequence's pages into ``out``."""
        call = self.bind_prefill_paged(q, k_cache, k_scale, v_cache, v_scale, v_zero, block_row, seq_len,
                                       pages_per_block, scale, out, workspace)
        if call is not None:
            call()

    def bind_prefill_paged(self, q, k_cache, k_scale, v_cache, v_scale, v_zero, block_row, seq_len: int,
                           pages_per_block: int, scale: float, out, workspace=None):
        """Validate one prefill; returns a :class:`BoundCall` (None when ``q_len`` is 0).

        ``workspace`` is a device buffer of at least :meth:`prefill_workspace_bytes`
        bytes; None allocates one (the prefill path is not graph-captured)."""
        _require(q.dim() == 3, "query [T,HQ,D]")
        head_dim = int(q.shape[2])
        _require(head_dim in (128, 256), "query [T,HQ,D] with D in (128, 256)")
        hkv = int(k_cache.shape[2]) if k_cache.dim() == 4 else -1
        _require(int(q.shape[1]) == GQA * hkv,
                 "query has %d heads, the K8/V4 cache holds %d (needs %d)" % (int(q.shape[1]), hkv, GQA * hkv))
        _checked_hkv(hkv)
        check_paged_k(k_cache, k_scale, hkv, head_dim)
        check_paged_v(v_cache, v_scale, v_zero, hkv, head_dim)
        q_len, seq_len = int(q.shape[0]), int(seq_len)
        if q_len > seq_len:
            raise RuntimeError("query longer than the KV sequence")
        if q_len == 0:
            return None
        _require(q.dtype in (torch.float16, torch.bfloat16), "query must be float16 or bfloat16")
        _require(q.stride(2) == 1 and q.stride(1) == head_dim, "query head/dim strides")
        _require(out.shape == q.shape, "out shape")
        _require(out.dtype in (torch.float16, torch.bfloat16, torch.float32), "out float16, bfloat16 or float32")
        _require(out.stride(2) == 1 and out.stride(1) == head_dim, "out head/dim strides")
        _require(block_row.dtype == torch.int32 and block_row.dim() == 1 and block_row.stride(0) == 1,
                 "block_row must be a contiguous int32 [width] row")
        _require(int(pages_per_block) >= 1, "pages_per_block")
        tensors = (q, k_cache, k_scale, v_cache, v_scale, v_zero, block_row, out)
        dev = _on_gpu(*tensors)
        need = self.prefill_workspace_bytes(seq_len, q_len, hkv, head_dim)
        if workspace is None:
            workspace = torch.empty(max(need, 16) // 4 + 4, dtype=torch.float32, device=dev)
        _require(workspace.is_contiguous() and workspace.device == dev, "prefill workspace must be a contiguous "
                 "buffer on the query's device")
        tensors = tensors + (workspace,)
        args = [
            _ptr(q), _DTYPE_CODE[q.dtype], int(q.stride(0)) if q_len > 1 else GQA * hkv * head_dim,
            *cache_args(k_cache, k_scale, v_cache, v_scale, v_zero),
            _ptr(block_row), int(block_row.shape[0]), int(pages_per_block), seq_len, q_len, hkv, head_dim,
            float(scale), _ptr(out), _DTYPE_CODE[out.dtype],
            int(out.stride(0)) if q_len > 1 else GQA * hkv * head_dim,
            _ptr(workspace), int(workspace.numel()) * workspace.element_size(),
        ]
        return BoundCall(self._lib, self._lib.k8v4_prefill_paged, args, dev, tensors)

    def prefill_batch_workspace_bytes(self, hkv: int, head_dim: int) -> int:
        """Scratch bytes :meth:`prefill_paged_batch` needs (any sequences)."""
        n = int(self._lib.k8v4_prefill_batch_workspace_bytes(int(hkv), int(head_dim)))
        _require(n >= 0, "bad shape for the prefill workspace")
        return n

    def prefill_paged_batch(self, q, k_cache, k_scale, v_cache, v_scale, v_zero, block_table, tok0, q_lens,
                            seq_lens, rows, pages_per_block: int, scale: float, out, workspace=None):
        """Several sequences' prefill in one call (the chunks of one step).

        Sequence i: query rows ``q[tok0[i] : tok0[i] + q_lens[i]]`` (bottom-right
        causal over its ``seq_lens[i]`` keys) into the same rows of ``out``, its
        pages in ``block_table[rows[i]]``.  ``tok0``, ``q_lens``, ``seq_lens`` and
        ``rows`` are Python integer sequences of one length.  Same numerics as
        :meth:`prefill_paged` per sequence."""
        _require(q.dim() == 3, "query [T,HQ,D]")
        head_dim = int(q.shape[2])
        _require(head_dim in (128, 256), "query [T,HQ,D] with D in (128, 256)")
        hkv = int(k_cache.shape[2]) if k_cache.dim() == 4 else -1
        _require(int(q.shape[1]) == GQA * hkv,
                 "query has %d heads, the K8/V4 cache holds %d (needs %d)" % (int(q.shape[1]), hkv, GQA * hkv))
        _checked_hkv(hkv)
        check_paged_k(k_cache, k_scale, hkv, head_dim)
        check_paged_v(v_cache, v_scale, v_zero, hkv, head_dim)
        tok0, q_lens, seq_lens, rows = ([int(x) for x in v] for v in (tok0, q_lens, seq_lens, rows))
        n = len(tok0)
        _require(len(q_lens) == n and len(seq_lens) == n and len(rows) == n,
                 "tok0, q_lens, seq_lens and rows must have one length")
        _require(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.stride(1) == 1,
                 "block_table must be int32 [B, W] with unit column stride")
        tokens = int(q.shape[0])
        for t0, ql, sl, r in zip(tok0, q_lens, seq_lens, rows):
            if ql > sl:
                raise RuntimeError("query longer than the KV sequence")
            _require(ql >= 0 and t0 >= 0 and t0 + ql <= tokens, "sequence rows outside the query")
            _require(0 <= r < int(block_table.shape[0]), "block table row out of range")
        if n == 0 or max(q_lens) == 0:
            return
        _require(q.dtype in (torch.float16, torch.bfloat16), "query must be float16 or bfloat16")
        _require(q.stride(2) == 1 and q.stride(1) == head_dim, "query head/dim strides")
        _require(out.shape == q.shape, "out shape")
        _require(out.dtype in (torch.float16, torch.bfloat16, torch.float32), "out float16, bfloat16 or float32")
        _require(out.stride(2) == 1 and out.stride(1) == head_dim, "out head/dim strides")
        _require(int(pages_per_block) >= 1, "pages_per_block")
        tensors = (q, k_cache, k_scale, v_cache, v_scale, v_zero, block_table, out)
        dev = _on_gpu(*tensors)
        need = self.prefill_batch_workspace_bytes(hkv, head_dim)
        if workspace is None:
            workspace = torch.empty(max(need, 16) // 4 + 4, dtype=torch.float32, device=dev)
        _require(workspace.is_contiguous() and workspace.device == dev, "prefill workspace must be a contiguous "
                 "buffer on the query's device")
        arrays = [(ctypes.c_int64 * n)(*v) for v in (tok0, q_lens, seq_lens, rows)]
        row_stride = GQA * hkv * head_dim
        rc = self._lib.k8v4_prefill_paged_batch(
            _ptr(q), _DTYPE_CODE[q.dtype], int(q.stride(0)) if tokens > 1 else row_stride,
            *cache_args(k_cache, k_scale, v_cache, v_scale, v_zero),
            _ptr(block_table), int(block_table.stride(0)), int(block_table.shape[1]), int(pages_per_block), n,
            *[ctypes.cast(x, ctypes.c_void_p) for x in arrays], hkv, head_dim, float(scale),
            _ptr(out), _DTYPE_CODE[out.dtype], int(out.stride(0)) if tokens > 1 else row_stride,
            _ptr(workspace), int(workspace.numel()) * workspace.element_size(), _stream(dev))
        _check(rc, self._lib)

    # -- K-only / V-only stores ----------------------------------------------
    def k_store_paged(self, k_fp16, slot_mapping, k_cache, k_scale):
        """The K half of :meth:`kv_store_paged` (xe2_kv_ops.cpp:1371-1389)."""
        _require(k_fp16.dim() == 3 and int(k_fp16.shape[2]) in (128, 256), "k_fp16 [T,HKV,D] with D in (128, 256)")
        head_dim = int(k_fp16.shape[2])
        _require(slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous(), "slot_mapping int64")
        hkv = _checked_hkv(int(k_fp16.shape[1]))
        check_paged_k(k_cache, k_scale, hkv, head_dim)
        _require(slot_mapping.numel() == k_fp16.shape[0], "slot_mapping [T]")
        ks = _src_rows(k_fp16, "k_fp16", hkv, head_dim)
        if k_fp16.shape[0] == 0:
            return
        dev = _on_gpu(k_fp16, slot_mapping, k_cache, k_scale)
        rc = self._lib.k8v4_k_store_paged(_ptr(k_fp16), _DTYPE_CODE[k_fp16.dtype], ks, _ptr(slot_mapping),
                                          int(k_fp16.shape[0]), hkv, head_dim, _ptr(k_cache), _ptr(k_scale),
                                          int(k_cache.shape[0]), int(k_cache.stride(0)), int(k_scale.stride(0)) * 4,
                                          _stream(dev))
        _check(rc, self._lib)

    def v_store_paged(self, v_fp16, slot_mapping, v_cache, v_scale, v_zero):
        """The V half of :meth:`kv_store_paged` (xe2_kv_ops.cpp:1391-1409)."""
        _require(v_fp16.dim() == 3 and int(v_fp16.shape[2]) in (128, 256), "v_fp16 [T,HKV,D] with D in (128, 256)")
        head_dim = int(v_fp16.shape[2])
        _require(slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous(), "slot_mapping int64")
        hkv = _checked_hkv(int(v_fp16.shape[1]))
        check_paged_v(v_cache, v_scale, v_zero, hkv, head_dim)
        _require(slot_mapping.numel() == v_fp16.shape[0], "slot_mapping [T]")
        vs = _src_rows(v_fp16, "v_fp16", hkv, head_dim)
        if v_fp16.shape[0] == 0:
            return
        dev = _on_gpu(v_fp16, slot_mapping, v_cache, v_scale, v_zero)
        rc = self._lib.k8v4_v_store_paged(_ptr(v_fp16), _DTYPE_CODE[v_fp16.dtype], vs, _ptr(slot_mapping),
                                          int(v_fp16.shape[0]), hkv, head_dim, _ptr(v_cache), _ptr(v_scale),
                                          _ptr(v_zero), int(v_cache.shape[0]), int(v_cache.stride(0)),
                                          int(v_scale.stride(0)) * 4, int(v_zero.stride(0)) * 4, _stream(dev))
        _check(rc, self._lib)

    # -- the Q-once tile and the ops that read it ----------------------------
    def q_quant_once(self, q_fp16, q8, q_scale):
        """Quantize the padded query tile ``[HKV, 64, D]`` into ``q8`` / ``q_scale`` (xe2_kv_ops.cpp:1248-1265)."""
        _require(q_fp16.dtype in (torch.float16, torch.bfloat16), "q_fp16 must be float16 or bfloat16")
        _require(q_fp16.dim() == 3 and q_fp16.shape[1] == PAGE and int(q_fp16.shape[2]) in (128, 256),
                 "q_fp16 shape [HKV,64,D]")
        _require(q_fp16.is_contiguous(), "q_fp16 must be contiguous")
        hkv = _checked_hkv(int(q_fp16.shape[0]))
        self._quantize_tile(q_fp16, Q_PADDED, 0, 0, hkv, int(q_fp16.shape[2]), q8, q_scale)

    def _quantize_tile(self, q, layout, tok_stride, ntok, hkv, head_dim, q8, q_scale):
        _require(q8.dtype == torch.int8, "q8 must be int8")
        _require(q_scale.dtype == torch.float32, "q_scale must be float32")
        _require(q8.is_contiguous() and q8.numel() == hkv * PAGE * head_dim, "q8 numel [HKV,64,D]")
        _require(q_scale.is_contiguous() and q_scale.numel() == hkv * PAGE, "q_scale numel [HKV,64]")
        dev = _on_gpu(q, q8, q_scale)
        rc = self._lib.k8v4_q_quant(_ptr(q), _DTYPE_CODE[q.dtype], layout, tok_stride, ntok, hkv, head_dim,
                                    _ptr(q8), _ptr(q_scale), _stream(dev))
        _check(rc, self._lib)

    def int8k_int4v_s1_paged(self, q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero, block_table, seq_lens,
                             out):
        """One sequence over the paged cache from a Q-once tile, workspace owned by
        the library (the reference's legacy op, xe2_kv_ops.cpp:1628-1639)."""
        self.int8k_int4v_s1_varlen_paged(q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero, block_table,
                                         seq_lens, None, None, None, None, None, out, 1)

    def int8k_int4v_s1_varlen_paged(self, q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero, block_table,
                                    seq_lens, visible_lens, partials_ws, m_ws, l_ws, merged_ws, out,
                                    pages_per_block: int = 1):
        """One sequence from a Q-once tile with optional explicit causal ends and a
        caller workspace (xe2_kv_ops.cpp:1641-1660).  ``out`` is ``[Tq, HQ, D]``;
        Tq is the query length.  ``m_ws``, ``l_ws`` and ``merged_ws`` are accepted
        and unused; ``partials_ws`` holds the split states (None: the library's
        own buffer, as the reference's legacy op keeps one)."""
        del m_ws, l_ws, merged_ws
        _require(q8.dtype == torch.int8, "q8 int8")
        _require(q_scale.dtype == torch.float32, "q_scale float32")
        _require(k_cache.dim() == 4, "k_cache [num_blocks,64,HKV,D] NHD")
        hkv = _checked_hkv(int(k_cache.shape[2]))
        head_dim = int(k_cache.shape[3])
        _require(head_dim in (128, 256), "k_cache head dim must be 128 or 256")
        check_paged_k(k_cache, k_scale, hkv, head_dim)
        check_paged_v(v_cache, v_scale, v_zero, hkv, head_dim)
        _require(k_cache.shape[0] == v_cache.shape[0], "k/v num_blocks")
        _require(q8.is_contiguous() and q8.numel() == hkv * PAGE * head_dim, "q8 unique [HKV,64,D]")
        _require(q_scale.is_contiguous() and q_scale.numel() == hkv * PAGE, "q_scale numel [HKV,64]")
        _require(block_table.dtype == torch.int32, "block_table int32")
        row = block_table if block_table.dim() == 1 else block_table.reshape(-1, block_table.shape[-1])[0]
        _require(row.numel() > 0 and row.is_contiguous(), "block_table n_splits")
        _require(seq_lens.dtype == torch.int32 and seq_lens.numel() >= 1 and seq_lens.is_contiguous(),
                 "seq_lens int32")
        _require(out.dim() == 3 and out.shape[1] == GQA * hkv and out.shape[2] == head_dim, "out [Tq,HQ,D]")
        _require(out.dtype in (torch.float16, torch.bfloat16, torch.float32), "out float32 or float16")
        _require(out.stride(2) == 1 and out.stride(1) == head_dim, "out head/dim strides")
        tq = int(out.shape[0])
        _require(tq > 0 and tq * GQA <= PAGE, "Tq*GQA must fit BM=64 pad")
        vis_ptr, vis_stride = 0, 0
        if visible_lens is not None and visible_lens.numel() > 0:
            _require(visible_lens.dtype == torch.int32 and visible_lens.numel() >= tq + 1 and
                     visible_lens.is_contiguous(), "visible_lens int32 [1+Tq]")
            vis_ptr, vis_stride = _ptr(visible_lens), tq + 1
        ppb = max(1, int(pages_per_block))
        dev = _on_gpu(q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero, row, seq_lens, out)
        need = self.attn_workspace_bytes(1, int(row.numel()), ppb, tq, hkv, head_dim)
        if partials_ws is None:
            ws = self._own_workspace(dev, need)
        else:
            _require(partials_ws.is_contiguous() and partials_ws.device == dev, "partials_ws must be a contiguous "
                     "buffer on the cache's device")
            ws = partials_ws
        rc = self._lib.k8v4_attn_batch_q8(
            _ptr(q8), _ptr(q_scale), hkv * PAGE * head_dim, hkv * PAGE,
            *cache_args(k_cache, k_scale, v_cache, v_scale, v_zero),
            _ptr(row), int(row.numel()), int(row.numel()), ppb, _ptr(seq_lens), vis_ptr, vis_stride, 1, tq, hkv,
            head_dim, _ptr(out), _DTYPE_CODE[out.dtype], int(out.stride(0)) if tq > 1 else GQA * hkv * head_dim,
            _ptr(ws), int(ws.numel()) * ws.element_size(), 0, _stream(dev))
        _check(rc, self._lib)

    def _own_workspace(self, dev, nbytes: int) -> torch.Tensor:
        """The library-owned split-state buffer of the workspace-free legacy op (grows on demand)."""
        have = self._legacy_ws.get(dev)
        if have is None or have.numel() * 4 < nbytes:
            have = self._legacy_ws[dev] = torch.empty(max(4, -(-nbytes // 4)), dtype=torch.int32, device=dev)
        return have

    def int8k_int4v_s1_varlen_from_q(self, q_fp16, q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero,
                                     block_table, seq_lens, visible_lens, partials_ws, m_ws, l_ws, merged_ws, out,
                                     pages_per_block: int = 1):
        """Quantize ``q_fp16`` into the Q-once tile (token rows ``[T, HQ, D]`` are
        packed, a padded ``[HKV, 64, D]`` tile is quantized as is), then
        :meth:`int8k_int4v_s1_varlen_paged` (xe2_kv_ops.cpp:1663-1712)."""
        _require(q_fp16.dtype in (torch.float16, torch.bfloat16), "q_fp16 must be float16 or bfloat16")
        _require(k_cache.dim() == 4, "k_cache [num_blocks,64,HKV,D] NHD")
        hkv = _checked_hkv(int(k_cache.shape[2]))
        head_dim = int(k_cache.shape[3])
        if q_fp16.dim() == 3 and q_fp16.shape[1] == GQA * hkv and q_fp16.shape[2] == head_dim:
            tq = int(q_fp16.shape[0])
            _require(tq > 0 and tq * GQA <= PAGE, "tq*GQA exceeds BM")
            _require(q_fp16.stride(2) == 1 and q_fp16.stride(1) == head_dim, "q_fp16 head/dim strides")
            self._quantize_tile(q_fp16, Q_TOKENS, int(q_fp16.stride(0)) if tq > 1 else GQA * hkv * head_dim, tq,
                                hkv, head_dim, q8, q_scale)
        else:
            _require(q_fp16.numel() == hkv * PAGE * head_dim and q_fp16.is_contiguous(), "q_fp16 numel")
            self._quantize_tile(q_fp16, Q_PADDED, 0, 0, hkv, head_dim, q8, q_scale)
        self.int8k_int4v_s1_varlen_paged(q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero, block_table,
                                         seq_lens, visible_lens, partials_ws, m_ws, l_ws, merged_ws, out,
                                         pages_per_block)

    def int8k_int4v_decode_step(self, q_fp16, k_fp16, v_fp16, slot_mapping, q8, q_scale, k_cache, k_scale, v_cache,
                                v_scale, v_zero, block_table, seq_lens, visible_lens, partials_ws, m_ws, l_ws,
                                merged_ws, out):
        """One decode step of one sequence: store the new K/V, then attend
        (xe2_kv_ops.cpp:1716-1731)."""
        self.kv_store_paged(k_fp16, v_fp16, slot_mapping, k_cache, k_scale, v_cache, v_scale, v_zero)
        self.int8k_int4v_s1_varlen_from_q(q_fp16, q8, q_scale, k_cache, k_scale, v_cache, v_scale, v_zero,
                                          block_table, seq_lens, visible_lens, partials_ws, m_ws, l_ws, merged_ws,
                                          out)

    # -- the reference's unpaged single-page stage tests ---------------------
    _UNPAGED = ("%s: the reference's unpaged single-page op (contiguous [64, 256] K/V rows, per-page partial "
                "outputs) is a stage test of its own kernels and is not part of this library; use %s")

    def k_store(self, *args, **kwargs):
        raise RuntimeError(self._UNPAGED % ("k_store", "k_store_paged or kv_store_paged"))

    def v_store(self, *args, **kwargs):
        raise RuntimeError(self._UNPAGED % ("v_store", "v_store_paged or kv_store_paged"))

    def int8k_int4v_s1(self, *args, **kwargs):
        raise RuntimeError(self._UNPAGED % ("int8k_int4v_s1", "int8k_int4v_s1_paged"))


def ops() -> _Ops:
    """The op table, after loading the library named by :func:`library_path`."""
    global _OPS
    lib = load_library()
    if _OPS is None or _OPS._lib is not lib:
        _OPS = _Ops(lib)
    return _OPS


__all__ = ["BoundCall", "GQA", "PAGE", "library_path", "load_library", "ops", "check_paged_k", "check_paged_v"]
