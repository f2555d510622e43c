"""The vLLM registration patch on stand-in ROCm vLLM trees (CPU only).

Mirrors the reference's patch test (k8v4_v030/tests/test_patch.py:39-65):
three edits applied once, a second run changes nothing, the edits sit where
the selector reads them, and a tree that lacks an anchor or carries an edit
twice fails loudly.  The stand-in files follow the shape of vLLM's own
``config/cache.py``, ``utils/torch_utils.py`` and ``platforms/rocm.py``; the
patched files are executed to check what the selector returns.
"""
from __future__ import annotations

import types
import typing
from pathlib import Path

import pytest
import torch

from k8v4_v030.layout import CACHE_DTYPE
from k8v4_v030.patch_installed_vllm import BACKEND_PATH, SELECTOR_MARK, main, patch_installed, patch_vllm_tree

CACHE = '''\
from typing import Literal

CacheDType = Literal[
    "auto",
    "bfloat16",
    "fp8",
    "fp8_e4m3",
    "fp8_e5m2",
]
'''

TORCH = '''\
import torch

STR_DTYPE_TO_TORCH_DTYPE = {
    "float32": torch.float32,
    "half": torch.half,
    "bfloat16": torch.bfloat16,
    "fp8": torch.uint8,
    "fp8_e4m3": torch.uint8,
}
'''

TRITON = "vllm.v1.attention.backends.triton_attn.TritonAttentionBackend"
ROCM_ATTN = "vllm.v1.attention.backends.rocm_attn.RocmAttentionBackend"

ROCM = '''\
class RocmPlatform:
    @classmethod
    def get_attn_backend_cls(cls, selected_backend, attn_selector_config, num_heads=None) -> str:
        """Picks the attention backend for this platform."""
        block_size = attn_selector_config.block_size
        kv_cache_dtype = attn_selector_config.kv_cache_dtype
        if kv_cache_dtype is not None and kv_cache_dtype.startswith("fp8"):
            return "%s"
        return "%s"
''' % (ROCM_ATTN, TRITON)

# An older selector signature: the cache dtype is a positional argument.
ROCM_OLD = '''\
class RocmPlatform:
    @classmethod
    def get_attn_backend_cls(cls, selected_backend, head_size, dtype, kv_cache_dtype, block_size, use_v1,
                             use_mla):
        if use_mla:
            return "mla"
        return "%s"
''' % TRITON


def make_tree(root: Path, cache=CACHE, torch_utils=TORCH, rocm=ROCM) -> Path:
    for rel, text in (("config/cache.py", cache), ("utils/torch_utils.py", torch_utils),
                      ("platforms/rocm.py", rocm)):
        path = root / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(text, encoding="utf-8")
    return root


def run_module(path: Path) -> dict:
    scope: dict = {"__name__": "patched"}
    exec(compile(path.read_text(encoding="utf-8"), str(path), "exec"), scope)  # noqa: S102 -- test-written file
    return scope


def select(scope: dict, kv_cache_dtype: str) -> str:
    cfg = types.SimpleNamespace(kv_cache_dtype=kv_cache_dtype, block_size=64)
    return scope["RocmPlatform"].get_attn_backend_cls(None, cfg)


def test_three_edits_apply_once(tmp_path):
    root = make_tree(tmp_path)
    assert patch_vllm_tree(root) == ["cache:patched", "torch_utils:patched", "rocm:patched"]
    assert patch_vllm_tree(root) == ["cache:unchanged", "torch_utils:unchanged", "rocm:unchanged"]
    cache = (root / "config/cache.py").read_text()
    torch_utils = (root / "utils/torch_utils.py").read_text()
    rocm = (root / "platforms/rocm.py").read_text()
    assert cache.count('"%s"' % CACHE_DTYPE) == 1 and torch_utils.count('"%s"' % CACHE_DTYPE) == 1
    assert rocm.count(SELECTOR_MARK) == 1 and rocm.count(BACKEND_PATH) == 1
    # The new dtype is the literal's last member; the map entry follows the existing ones.
    assert '"fp8_e5m2",\n    "%s",\n]' % CACHE_DTYPE in cache
    assert torch_utils.index('"fp8_e4m3"') < torch_utils.index('"%s"' % CACHE_DTYPE)
    # The selector's early return comes before any other selection, after the docstring.
    assert rocm.index('"""Picks') < rocm.index(SELECTOR_MARK) < rocm.index("block_size =")
    assert rocm.count('startswith("fp8")') == 1


def test_patched_files_run_and_select_the_backend(tmp_path):
    root = make_tree(tmp_path)
    patch_vllm_tree(root)
    assert CACHE_DTYPE in typing.get_args(run_module(root / "config/cache.py")["CacheDType"])
    assert run_module(root / "utils/torch_utils.py")["STR_DTYPE_TO_TORCH_DTYPE"][CACHE_DTYPE] is torch.uint8
    rocm = run_module(root / "platforms/rocm.py")
    assert select(rocm, CACHE_DTYPE) == BACKEND_PATH
    assert select(rocm, "auto") == TRITON and select(rocm, "fp8") == ROCM_ATTN


def test_positional_dtype_selector_and_one_line_collections(tmp_path):
    root = make_tree(tmp_path, cache='from typing import Literal\nCacheDType = Literal["auto", "fp8"]\n',
                     torch_utils='import torch\nSTR_DTYPE_TO_TORCH_DTYPE = {"half": torch.half}\n',
                     rocm=ROCM_OLD)
    assert patch_vllm_tree(root) == ["cache:patched", "torch_utils:patched", "rocm:patched"]
    assert typing.get_args(run_module(root / "config/cache.py")["CacheDType"]) == ("auto", "fp8", CACHE_DTYPE)
    assert run_module(root / "utils/torch_utils.py")["STR_DTYPE_TO_TORCH_DTYPE"] == {
        "half": torch.half, CACHE_DTYPE: torch.uint8}
    cls = run_module(root / "platforms/rocm.py")["RocmPlatform"]
    assert cls.get_attn_backend_cls(None, 128, None, CACHE_DTYPE, 64, True, False) == BACKEND_PATH
    assert cls.get_attn_backend_cls(None, 128, None, "auto", 64, True, False) == TRITON


def test_missing_anchor_and_double_edit_fail_loudly(tmp_path):
    root = make_tree(tmp_path / "a", rocm="class RocmPlatform:\n    pass\n")
    with pytest.raises(RuntimeError, match="get_attn_backend_cls"):
        patch_vllm_tree(root)
    root = make_tree(tmp_path / "b", torch_utils="import torch\n")
    with pytest.raises(RuntimeError, match="STR_DTYPE_TO_TORCH_DTYPE"):
        patch_vllm_tree(root)
    root = make_tree(tmp_path / "c")
    patch_vllm_tree(root)
    path = root / "platforms/rocm.py"
    text = path.read_text()
    path.write_text(text.replace(SELECTOR_MARK, SELECTOR_MARK + "\n        " + SELECTOR_MARK, 1))
    with pytest.raises(RuntimeError, match="present 2 times"):
        patch_vllm_tree(root)
    (tmp_path / "d").mkdir()
    with pytest.raises(RuntimeError, match="missing"):
        patch_vllm_tree(tmp_path / "d")


def test_command_line_patches_the_named_roots(tmp_path, capsys):
    roots = [make_tree(tmp_path / "x"), make_tree(tmp_path / "y")]
    assert main([str(r) for r in roots]) == 0
    out = capsys.readouterr().out.splitlines()
    assert len(out) == 6 and all(line.endswith(":patched") for line in out)
    assert all(n.endswith(":unchanged") for n in patch_installed(tuple(roots)))
    with pytest.raises(RuntimeError, match="no vLLM tree"):
        patch_installed((tmp_path / "nowhere",))
