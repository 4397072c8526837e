"""Per-request paged cache updates and the bulk completed-page quantizer.

HIP replacements of the Triton operators of
``scripts/benchmark_page_gauge_overheads.py`` (same names, arguments and
``ValueError`` messages):

* ``append_kv`` (:242-269) -- FP16 append at per-request (page, offset);
* ``append_finalize_page_gauge`` (:272-317) -- centered append without RoPE
  and completed-page INT8 finalize into the same page index;
* ``quantize_completed_kv_pages`` (:208-239) -- bulk quantizer used to build
  every prefix cache.
"""

from __future__ import annotations

import torch

from . import _capi

PAGE = 16
DIM = 128


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _all_cuda_contiguous(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("tensors must be contiguous CUDA tensors")


def quantize_completed_kv_pages(key, value, key_center, value_center, key_codes, value_codes,
                                key_scales, value_scales) -> None:
    if key.shape != value.shape or key.ndim != 4:
        raise ValueError("K and V must have identical [pages, 16, heads, 128] shapes")
    if key.shape[1] != PAGE or key.shape[-1] != DIM:
        raise ValueError("K and V must have shape [pages, 16, heads, 128]")
    if key_center.shape != (key.shape[2], DIM) or value_center.shape != key_center.shape:
        raise ValueError("centers must be [heads, 128]")
    if key.dtype != torch.float16 or key_codes.dtype != torch.int8 or key_scales.dtype != torch.float16:
        raise ValueError("K/V and centers must be float16, codes int8, scales float16")
    _all_cuda_contiguous(key, value, key_center, value_center, key_codes, value_codes, key_scales,
                         value_scales)
    _capi.call("pg_quantize_completed_kv_pages", key.data_ptr(), value.data_ptr(),
               key_center.data_ptr(), value_center.data_ptr(), key_codes.data_ptr(),
               value_codes.data_ptr(), key_scales.data_ptr(), value_scales.data_ptr(), key.shape[0],
               key.shape[2], _stream())


def _check_ids(key, page_ids, page_offsets) -> None:
    if page_ids.shape != (key.shape[0],) or page_offsets.shape != page_ids.shape:
        raise ValueError("page IDs and offsets must have one entry per request")
    if page_ids.dtype != torch.int32 or page_offsets.dtype != torch.int32:
        raise ValueError("page IDs and offsets must be int32")


def append_kv(key, value, key_pages, value_pages, page_ids, page_offsets) -> None:
    if key.shape != value.shape or key.ndim != 3 or key.shape[-1] != DIM:
        raise ValueError("K/V inputs must be identical [batch,heads,128] tensors")
    if key_pages.shape != value_pages.shape or key_pages.ndim != 4:
        raise ValueError("page caches must be identical [pages,16,heads,128] tensors")
    if key_pages.shape[1:] != (PAGE, key.shape[1], DIM):
        raise ValueError("page cache shape does not match K/V inputs")
    _check_ids(key, page_ids, page_offsets)
    _all_cuda_contiguous(key, value, key_pages, value_pages, page_ids, page_offsets)
    _capi.call("pg_append_kv", key.data_ptr(), value.data_ptr(), key_pages.data_ptr(),
               value_pages.data_ptr(), page_ids.data_ptr(), page_offsets.data_ptr(), key.shape[0],
               key.shape[1], key_pages.shape[0], _stream())


def append_finalize_page_gauge(key, value, key_center, value_center, exact_key_pages,
                               exact_value_pages, key_codes, value_codes, key_scales,
                               value_scales, page_ids, page_offsets) -> None:
    if key.shape != value.shape or key.ndim != 3 or key.shape[-1] != DIM:
        raise ValueError("K/V inputs must be identical [batch,heads,128] tensors")
    expected_pages = (exact_key_pages.shape[0], PAGE, key.shape[1], DIM)
    for tensor in (exact_key_pages, exact_value_pages, key_codes, value_codes):
        if tensor.shape != expected_pages:
            raise ValueError("all exact/code caches must be [pages,16,heads,128]")
    if key_center.shape != (key.shape[1], DIM) or value_center.shape != key_center.shape:
        raise ValueError("centers must be [heads,128]")
    if key_scales.shape != (exact_key_pages.shape[0], key.shape[1]):
        raise ValueError("key scales must be [pages,heads]")
    if value_scales.shape != key_scales.shape:
        raise ValueError("value scales must match key scales")
    _check_ids(key, page_ids, page_offsets)
    _all_cuda_contiguous(key, value, key_center, value_center, exact_key_pages, exact_value_pages,
                         key_codes, value_codes, key_scales, value_scales, page_ids, page_offsets)
    _capi.call("pg_append_finalize_page_gauge", key.data_ptr(), value.data_ptr(),
               key_center.data_ptr(), value_center.data_ptr(), exact_key_pages.data_ptr(),
               exact_value_pages.data_ptr(), key_codes.data_ptr(), value_codes.data_ptr(),
               key_scales.data_ptr(), value_scales.data_ptr(), page_ids.data_ptr(),
               page_offsets.data_ptr(), key.shape[0], key.shape[1], exact_key_pages.shape[0],
               _stream())
