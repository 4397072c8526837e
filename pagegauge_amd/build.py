"""Build libpagegauge_hip.so (gfx950) in-tree with hipcc.

The library is the C-ABI boundary declared in ``include/pagegauge_hip.h``.
Every kernel source is compiled for gfx950 only, with packed-FP32 code
generation disabled (``-packed-fp32-ops``).  The cache-update source is also
compiled with ``-ffp-contract=off`` because its FP16/FP32 arithmetic must
round operation by operation; the decode source keeps contraction enabled.

Alternative builds for measured design comparisons (``python -m
pagegauge_amd.build --variant NAME``) go to ``lib/variants/NAME/``; the
product never loads them:

* ``qk_valu``: the INT8 path's QK contraction on the VALU
  (``v_dot4_i32_i8`` over the same query digits, K rows re-laid through LDS)
  instead of the i8 MFMA; identical integer scores.
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
    "pg_plan.cpp": [],
    "pg_update.hip": ["-ffp-contract=off"],
    # the memory-clause scheduler keeps the partial kernel's page-group loads
    # together: measured 1-3 % faster (B1/49K, 16K, B8 ragged), same bits
    "pg_decode.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
    "pg_decoder.hip": [],
    "pg_probe.hip": [],
}


VARIANTS = {
    "qk_valu": {"pg_decode.hip": ["-DPG_QK_VALU=1"]},
}


def variant_library(name: str) -> Path:
    return PACKAGE / "lib" / "variants" / name / "libpagegauge_hip.so"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libpagegauge_hip.so")
    return path


def _compile(source: str, extra: list[str], build_dir: Path) -> Path:
    src = CSRC / source
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    if source.endswith(".cpp"):
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{ROOT / 'include'}", "-c", str(src),
               "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n{' '.join(cmd)}\n{result.stdout}\n{result.stderr}")
    return obj


def build(verbose: bool = False, variant: str | None = None) -> Path:
    """Compile every source and link the shared library; returns its path.

    ``variant`` names an alternative build from ``VARIANTS``."""
    build_dir, library, sources = BUILD, LIBRARY, dict(SOURCES)
    if variant is not None:
        if variant not in VARIANTS:
            raise ValueError(f"unknown variant {variant!r}; known: {sorted(VARIANTS)}")
        build_dir, library = BUILD / "variants" / variant, variant_library(variant)
        for source, flags in VARIANTS[variant].items():
            sources[source] = sources[source] + flags
    build_dir.mkdir(parents=True, exist_ok=True)
    library.parent.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 1)) as pool:
        objects = list(pool.map(lambda item: _compile(item[0], item[1], build_dir), sources.items()))
    tmp = library.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking failed:\n{' '.join(cmd)}\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, library)
    if verbose:
        print(f"built {library}")
    return library


if __name__ == "__main__":
    import argparse
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--variant", choices=sorted(VARIANTS), default=None)
    build(verbose=True, variant=parser.parse_args().variant)
    sys.exit(0)
