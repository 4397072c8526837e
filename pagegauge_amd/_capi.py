"""ctypes binding of ``libpagegauge_hip.so`` (C ABI: ``include/pagegauge_hip.h``).

The library is built in-tree by ``pagegauge_amd/build.py`` (``__graft_entry__.build``).
There is no fallback: if the library is missing or cannot be loaded every
operator raises, so a GPU run can never silently use another path.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "lib" / "libpagegauge_hip.so"
ABI_VERSION = 4

PG_OK = 0
PG_KV_INT8 = 0
PG_KV_FP16 = 1
PG_KV_HETEROGENEOUS = 2

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class DecodePlan(ctypes.Structure):
    """Mirror of ``pg_decode_plan_t``."""

    _fields_ = [
        ("batch_size", _i32),
        ("num_qo_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("page_size", _i32),
        ("primary_kind", _i32),
        ("has_tail", _i32),
        ("split_pages", _i32),
        ("tail_split_pages", _i32),
        ("num_items", _i32),
        ("num_items_primary", _i32),
        ("max_items_per_request", _i32),
        ("waves_per_block", _i32),
        ("closed_form", _i32),
        ("cf_tail_items", _i32),
        ("cf_tail_begin", _i32),
        ("cf_tail_pages", _i32),
        ("cf_primary_begin", _i32),
        ("cf_primary_pages", _i32),
        ("reserved", _i32),
        ("items_offset", _i64),
        ("item_ptr_offset", _i64),
        ("partial_offset", _i64),
        ("workspace_bytes", _i64),
    ]


# name -> (restype, argtypes); every symbol declared in include/pagegauge_hip.h
PROTOTYPES = {
    "pg_last_error": (ctypes.c_char_p, []),
    "pg_abi_version": (_i32, []),
    "pg_rope_append_fp16": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32,
                                   _i32, _i32, _i32, _p, _i64, _i32, _p]),
    "pg_rope_append_page_gauge": (_i32, [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p,
                                         _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32,
                                         _i32, _p, _i64, _i32, _p]),
    "pg_rope_append_page_gauge_positions": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p,
                                                   _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32,
                                                   _i32, _i32, _i32, _i32, _i32, _i64, _i32, _p]),
    "pg_rope_append_page_gauge_slots": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p,
                                               _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32,
                                               _i32, _i64, _i64, _i64, _i32, _p]),
    "pg_append_kv": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "pg_append_finalize_page_gauge": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32,
                                             _i32, _i32, _p]),
    "pg_quantize_completed_kv_pages": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p]),
    "pg_quantize_page_gauge": (_i32, [_p, _p, _p, _p, _i64, _i32, _p]),
    "pg_prefill_page_gauge": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64,
                                     _i32, _p]),
    "pg_token_major_centers_workspace_bytes": (_i64, [_i64, _i32]),
    "pg_token_major_centers": (_i32, [_p, _i64, _p, _i64, _i64, _i32, _p, _p, _p, _i64, _p]),
    "pg_token_major_centers_noalloc_max_bytes": (_i64, []),
    "pg_token_major_centers_noalloc": (_i32, [_p, _i64, _p, _i64, _i64, _i32, _p, _p, _p]),
    "pg_decode_workspace_bytes": (_i64, [_i32, _i32, _i64, _i64]),
    "pg_select_split_pages": (_i32, [_i64, _i32, _i32, _i32, _i32]),
    "pg_decode_plan": (_i32, [_p, _p, _i32, _i32, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32,
                              _i32, _i32, _p, _i64, ctypes.POINTER(DecodePlan), _p]),
    "pg_decode_plan_host": (_i32, [_p, _p, _i32, _i32, _p, _p, _i32, _i32, _i32, _i32, _i32,
                                   _i32, _i32, _i32, ctypes.POINTER(DecodePlan), _p, _i64, _p]),
    "pg_decode_run": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p,
                             _p, _p, _p, _i64, _p, _p, _f32, _p, _p]),
    "pg_decode_run_timed": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p, _p, _p, _p, _p,
                                   _p, _p, _p, _p, _p, _i64, _p, _p, _f32, _p, _p, _p, _p]),
    "pg_decode_run_partial": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p, _p, _p, _p, _p,
                                     _p, _p, _p, _p, _f32, _p, _p]),
    "pg_decode_run_partial_timed": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p, _p, _p,
                                           _p, _p, _p, _p, _p, _p, _f32, _p, _p, _p, _p]),
    "pg_decode_run_heterogeneous": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p, _p, _p,
                                           _p, _p, _p, _p, _p, _p, _i64, _p, _p, _f32, _p, _p]),
    "pg_decode_run_finalize": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p, _p, _p, _p,
                                      _p, _p, _p, _p, _p, _p, _i64, _p, _p, _f32, _p, _p, _i32,
                                      _i32, _p]),
    "pg_decode_run_heterogeneous_finalize": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p,
                                                    _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p,
                                                    _f32, _p, _p, _i32, _i32, _p]),
    "pg_decode_run_combine": (_i32, [ctypes.POINTER(DecodePlan), _p, _i64, _p, _p, _p, _p]),
    "pg_decoder_gemv": (_i32, [_p, _i32, _i32, _p, _i64, _i32, _p, _f32, _i32, _p, _i64, _p, _i64,
                               _i32, _p]),
    "pg_decoder_qkv_rope_append": (_i32, [_p, _i32, _p, _i64, _i32, _p, _f32, _i32, _i32, _p, _p,
                                          _i64, _i32, _p, _i32, _p, _p, _p, _p, _p, _i64, _i32,
                                          _i32, _i32, _p]),
    "pg_argmax_f32": (_i32, [_p, _i32, _i32, _i64, _p, _p]),
    "pg_merge_state_in_place": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "pg_exact_tail_merge_center": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                                          _i32, _f32, _p]),
}

# libpagegauge_bench.so (include/pagegauge_bench.h): bench.py's probes
BENCH_LIBRARY_PATH = LIBRARY_PATH.with_name("libpagegauge_bench.so")
BENCH_PROTOTYPES = {
    "pg_last_error": (ctypes.c_char_p, []),
    "pg_abi_version": (_i32, []),
    "pg_probe_linear_read": (_i32, [_p, _i64, _p, _i64, _i32, _p, _p, _p]),
    "pg_probe_page_walk": (_i32, [_p, _p, _p, _i32, _i32, _i32, _p, _i64, _p, _p, _p]),
    "pg_probe_decode_walk": (_i32, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p, _p,
                                    _p]),
}

# exported by the trace build of the product library only
TRACE_PROTOTYPES = {
    "pg_trace_set_buffer": (_i32, [_p, _i64]),
}

_lock = threading.Lock()
_library = None
_bench_library = None


class LibraryMissingError(RuntimeError):
    pass


def load_library(path, prototypes=None):
    """A ctypes handle of the library at ``path`` with every prototype set
    and its ABI checked (not cached; ``library()`` holds the product's).
    Alternative builds (``python -m pagegauge_amd.build --variant NAME``)
    load beside the product this way; the trace build also binds
    ``pg_trace_set_buffer``."""
    if not Path(path).exists():
        raise LibraryMissingError(
            f"{path} is missing: build it with `python -c "
            "'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(path))
    table = dict(PROTOTYPES if prototypes is None else prototypes)
    if prototypes is None and hasattr(lib, "pg_trace_set_buffer"):
        table.update(TRACE_PROTOTYPES)
    for name, (restype, argtypes) in table.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.pg_abi_version()
    if version != ABI_VERSION:
        raise LibraryMissingError(
            f"{Path(path).name} ABI {version} does not match the bindings ({ABI_VERSION})")
    return lib


def library():
    """Load (once) and return the ctypes handle; raises if the build is absent."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is None:
            _library = load_library(LIBRARY_PATH)
    return _library


def bench_library():
    """Load (once) and return bench.py's probe library (libpagegauge_bench.so)."""
    global _bench_library
    if _bench_library is not None:
        return _bench_library
    with _lock:
        if _bench_library is None:
            _bench_library = load_library(BENCH_LIBRARY_PATH, BENCH_PROTOTYPES)
    return _bench_library


def last_error() -> str:
    return library().pg_last_error().decode("utf-8", "replace")


def check(rc: int, what: str) -> None:
    """Raise RuntimeError carrying the library's message for a failing call."""
    if rc != PG_OK:
        raise RuntimeError(f"{what}: {last_error()} (code {rc})")


def call(name: str, *args) -> None:
    check(getattr(library(), name)(*args), name)
