"""ctypes binding of the C restatement ``oracle/pg_oracle.c``.

TEST INFRASTRUCTURE ONLY (tests/, smoke() and bench.py's CPU baseline).
The library is built by ``oracle/Makefile`` into ``oracle/_build``.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "_build" / "libpg_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def library():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        p = ctypes.c_void_p
        lib.pgo_rope_rotate.argtypes = [p, p, p, p, ctypes.c_int64]
        lib.pgo_finalize_page.argtypes = [p, ctypes.c_int, p, p]
        lib.pgo_quantize_completed.argtypes = [p, p, ctypes.c_int64, ctypes.c_int, p, p]
        lib.pgo_double_to_half.argtypes = [ctypes.c_double]
        lib.pgo_double_to_half.restype = ctypes.c_uint16
        lib.pgo_decode_page_gauge.argtypes = [
            p, ctypes.c_int, ctypes.c_int, ctypes.c_int, p, p, p, p, p, p, p,
            p, p, p, p, p, p, ctypes.c_int, ctypes.c_float, p, p]
        _lib = lib
    return _lib


def _ptr(array: np.ndarray | None):
    if array is None:
        return None
    assert array.flags["C_CONTIGUOUS"]
    return array.ctypes.data_as(ctypes.c_void_p)


def double_to_half_bits(value: float) -> int:
    return int(library().pgo_double_to_half(float(value)))


def rope_rotate(x: np.ndarray, cosine: np.ndarray, sine: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16)
    out = np.empty_like(x)
    library().pgo_rope_rotate(_ptr(x), _ptr(np.ascontiguousarray(cosine, np.float16)),
                              _ptr(np.ascontiguousarray(sine, np.float16)), _ptr(out),
                              x.size // 128)
    return out


def finalize_page(page: np.ndarray):
    """page [16, H, 128] fp16 -> (codes int8 same shape, scales fp16 [H])."""
    page = np.ascontiguousarray(page, dtype=np.float16)
    heads = page.shape[1]
    codes = np.empty(page.shape, dtype=np.int8)
    scales = np.empty((heads,), dtype=np.float16)
    library().pgo_finalize_page(_ptr(page), heads, _ptr(codes), _ptr(scales))
    return codes, scales


def quantize_completed(values: np.ndarray, center: np.ndarray):
    values = np.ascontiguousarray(values, dtype=np.float16)
    pages, _, heads, _ = values.shape
    codes = np.empty(values.shape, dtype=np.int8)
    scales = np.empty((pages, heads), dtype=np.float16)
    library().pgo_quantize_completed(_ptr(values), _ptr(np.ascontiguousarray(center, np.float16)),
                                     pages, heads, _ptr(codes), _ptr(scales))
    return codes, scales


def decode_page_gauge(query, k_codes, v_codes, k_scale, v_scale, indptr, indices, last_page_len,
                      sm_scale, tail_k=None, tail_v=None, tail_indptr=None, tail_indices=None,
                      tail_last_len=None, value_center=None):
    """Dense float32 decode of ``pg_oracle.c`` (INT8 pages + optional FP16 tail)."""
    query = np.ascontiguousarray(query, np.float16)
    batch, hq, _ = query.shape
    hkv = k_codes.shape[2]
    out = np.empty((batch, hq, 128), dtype=np.float16)
    lse = np.empty((batch, hq), dtype=np.float32)
    i32 = lambda a: None if a is None else np.ascontiguousarray(a, np.int32)  # noqa: E731
    f16 = lambda a: None if a is None else np.ascontiguousarray(a, np.float16)  # noqa: E731
    center = f16(value_center)
    keep = [query, np.ascontiguousarray(k_codes), np.ascontiguousarray(v_codes), f16(k_scale),
            f16(v_scale), i32(indptr), i32(indices), i32(last_page_len), f16(tail_k), f16(tail_v),
            i32(tail_indptr), i32(tail_indices), i32(tail_last_len), center]
    library().pgo_decode_page_gauge(
        _ptr(keep[0]), batch, hq, hkv, *[_ptr(a) for a in keep[1:]],
        int(center is not None and center.ndim == 3), float(sm_scale), _ptr(out), _ptr(lse))
    return out, lse
