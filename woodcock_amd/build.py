"""Build libwoodcock_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

    python -m woodcock_amd.build                 # compiles every csrc/*.hip, links the .so
    python -m woodcock_amd.build --incremental   # only sources older than their object

Objects go to woodcock_amd/_build/ (git-ignored); the shared library lands next
to this file so it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libwoodcock_hip.so"
ROOT_HEADER = PKG.parent / "include" / "woodcock_hip.h"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed-FP32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, incremental: bool = False) -> Path:
    obj = BUILD / (src.stem + ".o")
    if incremental and obj.exists():
        newest = max(p.stat().st_mtime for p in [src, *CSRC.glob("*.h"), ROOT_HEADER])
        if obj.stat().st_mtime > newest:
            return obj
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
    return obj


def build(jobs: int | None = None, incremental: bool = False) -> Path:
    """Compile every kernel source and link the shared library; returns its path.
    incremental: keep objects newer than their source and every header."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda p: _compile(p, incremental), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(incremental="--incremental" in sys.argv[1:])
    print(path, file=sys.stderr)
