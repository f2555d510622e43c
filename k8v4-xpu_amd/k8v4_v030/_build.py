"""Compile the HIP sources into the in-tree shared library (gfx950 only).

``python -m k8v4_v030._build`` (with ``k8v4-xpu_amd`` on ``sys.path``) or
``build()`` from Python.  Every ``csrc/*.hip`` file is compiled to an object
with hipcc, then linked into ``k8v4_v030/libk8v4_hip.so``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent  # k8v4-xpu_amd/
CSRC = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libk8v4_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "--offload-arch=" + ARCH,
    # Keep hipcc from forming packed-fp32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
# The store reproduces float64 rounding step for step: no fused multiply-adds.
# The decode kernels never produce or consume NaN (unwritten tails are masked
# by selection before any arithmetic), so max/min need no NaN quieting.
PER_FILE_FLAGS = {"kv_store.hip": ["-ffp-contract=off"], "q_quant.hip": ["-ffp-contract=off"],
                  "decode.hip": ["-fno-honor-nans"], "prefill.hip": ["-fno-honor-nans"]}


def hipcc() -> str:
    exe = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return exe


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    log = " ".join(cmd) + "\n" + proc.stdout + proc.stderr
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src.name, log))
    return obj, log


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link the library; returns its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources under %s" % CSRC)
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    workers = jobs or min(len(sources), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [pool.submit(_compile, s, BUILD_DIR / (s.stem + ".o")) for s in sources]
        for fut in futures:
            obj, log = fut.result()
            objs.append(obj)
            if verbose:
                print(log, file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "--offload-arch=" + ARCH, *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
