"""Build ``libmsgl_attn.so`` (gfx950) from ``csrc/`` with hipcc, in-tree.

Usage: ``python -m minisgl_hip._build`` (from ``mini-sglang-mlx_amd/``) or
``minisgl_hip._build.build()``. Every call recompiles; objects go to
``mini-sglang-mlx_amd/_build/`` and the library next to this file.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent  # mini-sglang-mlx_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD = ROOT / "_build"
LIB_NAME = "libmsgl_attn.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = os.environ.get("MSGL_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops are kept out of every kernel on this hardware
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources():
    """csrc/*.hip, *.cpp and csrc/inst/*.hip (the kernel instantiations of one
    (query, pool) type pair per file, so the largest units compile in parallel);
    largest first, so the pool starts the longest compiles first."""
    srcs = list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")) + list((CSRC / "inst").glob("*.hip"))
    return sorted(srcs, key=lambda f: (f.parent.name != "inst", f.name))


def object_path(src: Path) -> Path:
    """The object file of one source: its path under csrc/ joined by "_", so
    csrc/inst/decode_bf16.hip and a csrc/decode_bf16.hip would not collide."""
    return BUILD / ("_".join(src.relative_to(CSRC).parts) + ".o")


def _compile(src: Path, extra):
    obj = object_path(src)
    cmd = [HIPCC, *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False, extra_flags=()) -> Path:
    """Compile every source in csrc/ and link LIB_PATH. Returns the library path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, list(extra_flags)), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
