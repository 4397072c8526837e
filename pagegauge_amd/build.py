"""Build libpagegauge_hip.so (gfx950) in-tree with hipcc.

The library is the C-ABI boundary declared in ``include/pagegauge_hip.h``.
Every kernel source is compiled for gfx950 only, with packed-FP32 code
generation disabled (``-packed-fp32-ops``).  The cache-update source is also
compiled with ``-ffp-contract=off`` because its FP16/FP32 arithmetic must
round operation by operation; the decode source keeps contraction enabled.

``bench`` builds ``lib/libpagegauge_bench.so`` (``include/pagegauge_bench.h``):
bench.py's HBM read probes, measurement helpers outside the product ABI.

Alternative builds of the product for measured design comparisons are built
on request only (``python -m pagegauge_amd.build --variant NAME``) into
``lib/variants/NAME/``; the product never loads them, and each carries a
digest of the sources and flags it was built from (``variant_is_current``):

* ``qk_valu``: the INT8 path's QK contraction on the VALU
  (``v_dot4_i32_i8`` over the same query digits, K rows re-laid through LDS)
  instead of the i8 MFMA; identical integer scores;
* ``trace``: the product with the partial kernel's per-wave phase trace
  compiled in (``-DPG_TRACE=1``, ``pg_trace_set_buffer``; bench.py --trace);
* ``trace_conditional_scales``: the trace build with the page-scale loads in
  their earlier conditional form (bench.py --trace's before/after);
* ``default_scheduler``: the product with the decode source under LLVM's
  default machine scheduler instead of the memory-clause strategy;
* ``interleaved_heads``: the KV heads of an item's two workgroups
  interleaved (even, odd) instead of in blocks (0-3, 4-7);
* ``full_line_k``: whole 128-byte K rows per load instruction, the MFMA
  operand handed over by a DPP rotation.
"""

from __future__ import annotations

import hashlib
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
BENCH_LIBRARY = PACKAGE / "lib" / "libpagegauge_bench.so"
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
    # together: about 1 % faster from 16K tokens up (the default_scheduler
    # variant against it), same output bits
    "pg_decode.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
    "pg_decoder.hip": [],
}

BENCH_SOURCES = {
    "pg_error.cpp": [],
    "pg_probe.hip": [],
}

VARIANTS = {
    "qk_valu": {"pg_decode.hip": ["-DPG_QK_VALU=1"]},
    "trace": {"pg_decode.hip": ["-DPG_TRACE=1"]},
    "trace_conditional_scales": {"pg_decode.hip": ["-DPG_TRACE=1",
                                                   "-DPG_CONDITIONAL_SCALE_LOADS=1"]},
    # None: the source's own flags are dropped, not extended
    "default_scheduler": {"pg_decode.hip": None},
    "interleaved_heads": {"pg_decode.hip": ["-DPG_INTERLEAVED_HEADS=1"]},
    "full_line_k": {"pg_decode.hip": ["-DPG_FULL_LINE_K=1"]},
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


def _digest(sources: dict) -> str:
    """Digest of the headers, the sources and their flags (paths left out, so
    that a tree copied elsewhere gives the same digest)."""
    h = hashlib.sha256()
    headers = sorted(CSRC.glob("*.h")) + sorted((ROOT / "include").glob("*.h"))
    for path in headers:
        h.update(path.name.encode() + b"\0" + path.read_bytes())
    for name, flags in sorted(sources.items()):
        h.update(name.encode() + b"\0" + (CSRC / name).read_bytes() + " ".join(flags).encode())
    return h.hexdigest()


def _digest_file(library: Path) -> Path:
    return library.with_name(library.name + ".digest")


def _link(sources: dict, build_dir: Path, library: Path, verbose: bool) -> Path:
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
    _digest_file(library).write_text(_digest(sources) + "\n")
    if verbose:
        print(f"built {library}")
    return library


def variant_sources(variant: str) -> dict:
    if variant not in VARIANTS:
        raise ValueError(f"unknown variant {variant!r}; known: {sorted(VARIANTS)}")
    sources = dict(SOURCES)
    for source, flags in VARIANTS[variant].items():
        sources[source] = [] if flags is None else sources[source] + flags
    return sources


def variant_is_current(variant: str) -> bool:
    """The variant's library exists and was built from today's sources and flags."""
    library = variant_library(variant)
    digest = _digest_file(library)
    return (library.exists() and digest.exists()
            and digest.read_text().strip() == _digest(variant_sources(variant)))


def build(verbose: bool = False, variant: str | None = None) -> Path:
    """Compile every source and link the shared library; returns its path.

    ``variant`` names an alternative build from ``VARIANTS``."""
    if variant is None:
        return _link(dict(SOURCES), BUILD, LIBRARY, verbose)
    return _link(variant_sources(variant), BUILD / "variants" / variant, variant_library(variant),
                 verbose)


def build_bench(verbose: bool = False) -> Path:
    """bench.py's measurement helpers (``include/pagegauge_bench.h``)."""
    return _link(dict(BENCH_SOURCES), BUILD / "bench", BENCH_LIBRARY, verbose)


if __name__ == "__main__":
    import argparse
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--variant", choices=sorted(VARIANTS), default=None)
    parser.add_argument("--bench", action="store_true", help="the bench-only probe library")
    args = parser.parse_args()
    if args.bench:
        build_bench(verbose=True)
    else:
        build(verbose=True, variant=args.variant)
    sys.exit(0)
