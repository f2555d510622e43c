"""Register the ``int8_k_int4_v`` cache dtype and this backend in an installed
vLLM tree for the ROCm platform.

Reference: k8v4_v030/patch_installed_vllm.py:12-30, :107-138 (the same three
registrations against vLLM's XPU platform file).  Three edits per vLLM package
root, each applied at most once:

* ``config/cache.py``: ``"int8_k_int4_v"`` joins the ``CacheDType`` literal;
* ``utils/torch_utils.py``: ``"int8_k_int4_v": torch.uint8`` joins
  ``STR_DTYPE_TO_TORCH_DTYPE`` (the cache is a byte allocation);
* ``platforms/rocm.py``: ``get_attn_backend_cls`` returns
  ``k8v4_v030.backend.Xe2K8V4AttentionBackend`` for that cache dtype before
  any other selection.

The edit points are found from the files' syntax trees rather than from fixed
text, so the patch applies to any vLLM release whose files keep these three
definitions.  A file that lacks one raises ``RuntimeError`` naming it; a file
that already carries the edit is left alone ("unchanged"); a file that carries
it more than once (a bad manual merge) raises.  Nothing is imported from the
vLLM tree, so patching never runs vLLM code.

Command line: ``python -m k8v4_v030.patch_installed_vllm [VLLM_ROOT ...]``;
without arguments every root that ``import vllm`` could resolve is patched.
"""
from __future__ import annotations

import ast
import importlib.util
import sys
from pathlib import Path

from .layout import CACHE_DTYPE

BACKEND_PATH = "k8v4_v030.backend.Xe2K8V4AttentionBackend"
# Marker of the selector edit (also the first line of the inserted block).
SELECTOR_MARK = "# k8v4: int8-K / int4-V paged cache"


def _find_assign(tree: ast.Module, name: str) -> ast.expr:
    for node in ast.walk(tree):
        targets = []
        if isinstance(node, ast.Assign):
            targets = node.targets
        elif isinstance(node, ast.AnnAssign) and node.value is not None:
            targets = [node.target]
        for t in targets:
            if isinstance(t, ast.Name) and t.id == name:
                return node.value
    raise LookupError(name)


def _insert_before_close(text: str, close_line: int, close_col: int, item: str) -> str:
    """Adds ``item`` as the last element of a bracketed collection whose closing
    bracket sits at (1-based line, 0-based column); keeps one element per line
    when the bracket has a line of its own."""
    lines = text.splitlines(keepends=True)
    line = lines[close_line - 1]
    head = line[:close_col]
    if head.strip() == "":
        # Closing bracket on its own line: a new line indented like the last element.
        prev = lines[close_line - 2] if close_line >= 2 else ""
        indent = prev[: len(prev) - len(prev.lstrip())] or head + "    "
        if prev.rstrip() and not prev.rstrip().endswith((",", "[", "{", "(")):
            lines[close_line - 2] = prev.rstrip("\n").rstrip() + ",\n"
        lines.insert(close_line - 1, "%s%s,\n" % (indent, item))
    else:
        stripped = head.rstrip()
        sep = "" if stripped.endswith((",", "[", "{")) else ", "
        lines[close_line - 1] = stripped + sep + item + line[close_col:]
    return "".join(lines)


def _patch_collection(path: Path, name: str, marker: str, item: str) -> str:
    text = path.read_text(encoding="utf-8")
    n = text.count(marker)
    if n == 1:
        return "unchanged"
    if n > 1:
        raise RuntimeError("%s: marker %r present %d times, expected at most once" % (path, marker, n))
    try:
        value = _find_assign(ast.parse(text), name)
    except LookupError:
        raise RuntimeError("%s is missing the %s definition" % (path, name)) from None
    # Literal[...] (a subscript) or a dict / list display: either way its last
    # character is the closing bracket the new element goes in front of.
    if not isinstance(value, (ast.Subscript, ast.Dict, ast.List)):
        raise RuntimeError("%s: %s is not a literal collection" % (path, name))
    close_line, close_col = value.end_lineno, value.end_col_offset - 1
    new = _insert_before_close(text, close_line, close_col, item)
    ast.parse(new)  # the edit must leave valid Python
    path.write_text(new, encoding="utf-8")
    return "patched"


def _selector_function(tree: ast.Module) -> ast.FunctionDef:
    for node in ast.walk(tree):
        if isinstance(node, ast.FunctionDef) and node.name == "get_attn_backend_cls":
            return node
    raise LookupError("get_attn_backend_cls")


def _patch_selector(path: Path) -> str:
    text = path.read_text(encoding="utf-8")
    n = text.count(SELECTOR_MARK)
    if n == 1:
        return "unchanged"
    if n > 1:
        raise RuntimeError("%s: marker %r present %d times, expected at most once" % (path, SELECTOR_MARK, n))
    try:
        fn = _selector_function(ast.parse(text))
    except LookupError:
        raise RuntimeError("%s is missing get_attn_backend_cls" % path) from None
    params = [a.arg for a in fn.args.args + fn.args.kwonlyargs]
    if "attn_selector_config" in params:
        dtype_expr = 'getattr(attn_selector_config, "kv_cache_dtype", None)'
    elif "kv_cache_dtype" in params:
        dtype_expr = "kv_cache_dtype"
    else:
        raise RuntimeError("%s: get_attn_backend_cls takes neither attn_selector_config nor kv_cache_dtype" % path)
    body = fn.body
    first = body[1] if (len(body) > 1 and isinstance(body[0], ast.Expr) and isinstance(
        getattr(body[0], "value", None), ast.Constant) and isinstance(body[0].value.value, str)) else body[0]
    lines = text.splitlines(keepends=True)
    at = first.lineno - 1
    indent = lines[at][: len(lines[at]) - len(lines[at].lstrip())]
    block = [
        "%s%s\n" % (indent, SELECTOR_MARK),
        '%sif %s == "%s":\n' % (indent, dtype_expr, CACHE_DTYPE),
        '%s    return "%s"\n' % (indent, BACKEND_PATH),
    ]
    new = "".join(lines[:at] + block + lines[at:])
    ast.parse(new)
    path.write_text(new, encoding="utf-8")
    return "patched"


def patch_vllm_tree(root: Path) -> list[str]:
    """Patches one vLLM package root; returns ``label:patched|unchanged`` per file."""
    root = Path(root)
    jobs = (
        ("cache", root / "config" / "cache.py",
         lambda p: _patch_collection(p, "CacheDType", '"%s"' % CACHE_DTYPE, '"%s"' % CACHE_DTYPE)),
        ("torch_utils", root / "utils" / "torch_utils.py",
         lambda p: _patch_collection(p, "STR_DTYPE_TO_TORCH_DTYPE", '"%s"' % CACHE_DTYPE,
                                     '"%s": torch.uint8' % CACHE_DTYPE)),
        ("rocm", root / "platforms" / "rocm.py", _patch_selector),
    )
    notes = []
    for label, path, fn in jobs:
        if not path.is_file():
            raise RuntimeError("missing %s" % path)
        notes.append("%s:%s" % (label, fn(path)))
    return notes


def default_roots() -> tuple[Path, ...]:
    """The vLLM package ``import vllm`` would load (found without importing it)."""
    spec = importlib.util.find_spec("vllm")
    if spec is None or not spec.submodule_search_locations:
        return ()
    return tuple(Path(p) for p in spec.submodule_search_locations)


def patch_installed(roots: tuple[Path, ...] | None = None) -> list[str]:
    roots = default_roots() if roots is None else roots
    notes = []
    for root in roots:
        if (Path(root) / "config" / "cache.py").is_file():
            notes.extend("%s %s" % (root, item) for item in patch_vllm_tree(Path(root)))
    if not notes:
        raise RuntimeError("no vLLM tree found")
    return notes


def main(argv: list[str]) -> int:
    roots = tuple(Path(a) for a in argv) if argv else None
    for line in patch_installed(roots):
        print(line)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
