"""Build libpagegauge_hip.so (gfx950) in-tree with hipcc.

The library is the C-ABI boundary declared in ``include/pagegauge_hip.h``.
Every kernel source is compiled for gfx950 only, with packed-FP32 code
generation disabled (``-packed-fp32-ops``).  The cache-update source is also
compiled with ``-ffp-contract=off`` because its FP16/FP32 arithmetic must
round operation by operation; the decode source keeps contraction enabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "lib" / "libpagegauge_hip.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]

SOURCES = {
    "pg_error.cpp": [],
    "pg_update.hip": ["-ffp-contract=off"],
    "pg_decode.hip": [],
    "pg_decoder.hip": [],
    "pg_probe.hip": [],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libpagegauge_hip.so")
    return path


def _compile(source: str, extra: list[str]) -> Path:
    src = CSRC / source
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    if source.endswith(".cpp"):
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{ROOT / 'include'}", "-c", str(src),
               "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n{' '.join(cmd)}\n{result.stdout}\n{result.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    BUILD.mkdir(parents=True, exist_ok=True)
    LIBRARY.parent.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as pool:
        objects = list(pool.map(lambda item: _compile(*item), SOURCES.items()))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking failed:\n{' '.join(cmd)}\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
