"""Builds libxfold_hip.so in-tree (xfold_cpu_amd/lib/) with hipcc for gfx950.

Usage: ``python -m xfold_cpu_amd._build`` (or ``__graft_entry__.build()``). Every call
recompiles; objects go to ``_build/`` at the repository root.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
LIBDIR = PACKAGE / "lib"
OBJDIR = ROOT / "_build"
LIBRARY = LIBDIR / "libxfold_hip.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
# Packed fp32 VALU ops are disabled for every kernel (they have given silently wrong
# results on these boxes); hipcc's host pass warns that it does not know the feature.
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    noisy = [line for line in proc.stderr.splitlines()
             if line.strip() and "packed-fp32-ops" not in line]
    if noisy:
        sys.stderr.write(f"[{src.name}]\n" + "\n".join(noisy) + "\n")
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY.relative_to(ROOT)} from {len(srcs)} sources")
    return LIBRARY


if __name__ == "__main__":
    build()
