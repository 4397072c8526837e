"""Drop-in for the PageGauge append extension (``load_append_extension``).

Mirrors ``scripts/page_gauge_runtime.py:16-29`` and the five pybind entry
points of ``tests/page_gauge_append_extension.cu:1030-1040`` (same names,
positional signatures, in-place semantics and ``RuntimeError`` messages), plus
``rope_append_page_gauge_positions`` for per-request positions.  Tensor-level
validation happens here; the kernels run through the C ABI of
``libpagegauge_hip.so`` on the current HIP stream.  Nothing is allocated and
nothing synchronises, so the calls are graph-capturable.
"""

from __future__ import annotations

import torch

from . import _capi

HEAD_DIM = 128
PAGE_SIZE = 16


def _fail(message: str) -> None:
    raise RuntimeError(message)


def _require(condition: bool, message: str) -> None:
    if not condition:
        _fail(message)


def _check_tensor(tensor: torch.Tensor, name: str, dtype: torch.dtype, dims: int) -> None:
    # tests/page_gauge_append_extension.cu:23-32
    _require(tensor.is_cuda, f"{name} must be CUDA")
    _require(tensor.dtype == dtype, f"{name} has the wrong dtype")
    _require(tensor.dim() == dims, f"{name} has the wrong rank")
    _require(tensor.is_contiguous(), f"{name} must be contiguous")


def _check_head_major(tensor: torch.Tensor, name: str) -> None:
    # tests/page_gauge_append_extension.cu:34-41
    _require(tensor.is_cuda, f"{name} must be CUDA")
    _require(tensor.dtype == torch.float16, f"{name} must be FP16")
    _require(tensor.dim() == 3, f"{name} must have rank three")
    _require(tensor.stride(2) == 1 and tensor.stride(1) == HEAD_DIM,
             f"{name} must be head-major with a contiguous head dimension")
    _require(tensor.data_ptr() % 4 == 0 and tensor.stride(0) % 2 == 0,
             f"{name} rows must be 4-byte aligned")


def _qkv_checks(query, key, value, rotated_query) -> None:
    _require(query.size(0) > 0 and query.size(0) == key.size(0) and query.size(0) == value.size(0),
             "Q/K/V batch sizes must match and be positive")
    _require(query.size(2) == HEAD_DIM and key.size(2) == HEAD_DIM and value.size(2) == HEAD_DIM,
             "head dimension must be 128")
    _require(key.shape == value.shape, "K/V input shapes must match")
    _require(rotated_query.shape == query.shape, "rotated query shape mismatch")


def _check_common(query, key, value, cosine, sine, rotated_query, key_pages, value_pages,
                  position: int) -> None:
    # tests/page_gauge_append_extension.cu:585-621
    _check_head_major(query, "query")
    _check_head_major(key, "key")
    _check_head_major(value, "value")
    _check_tensor(cosine, "cosine", torch.float16, 1)
    _check_tensor(sine, "sine", torch.float16, 1)
    _check_tensor(rotated_query, "rotated_query", torch.float16, 3)
    _check_tensor(key_pages, "key_pages", torch.float16, 4)
    _check_tensor(value_pages, "value_pages", torch.float16, 4)
    _qkv_checks(query, key, value, rotated_query)
    _require(cosine.numel() == HEAD_DIM and sine.numel() == HEAD_DIM,
             "RoPE vectors must contain 128 values")
    _require(key_pages.shape == value_pages.shape, "K/V page shapes must match")
    _require(key_pages.size(1) == PAGE_SIZE and key_pages.size(2) == key.size(1)
             and key_pages.size(3) == HEAD_DIM, "page cache must be NHD [pages,16,Hkv,128]")
    _require(position >= 0, "position must be non-negative")


def _check_dynamic(query, cosine, sine, position) -> None:
    # tests/page_gauge_append_extension.cu:623-640
    _check_tensor(cosine, "cosine", torch.float16, 2)
    _check_tensor(sine, "sine", torch.float16, 2)
    _check_tensor(position, "position", torch.int32, 1)
    _require(cosine.shape == sine.shape and cosine.size(0) > 0 and cosine.size(1) == HEAD_DIM,
             "dynamic RoPE tables must be matching [positions,128] tensors")
    _require(position.numel() == 1, "dynamic position must contain exactly one int32 scalar")
    _require(cosine.get_device() == query.get_device() and sine.get_device() == query.get_device()
             and position.get_device() == query.get_device(),
             "dynamic position, RoPE tables, and Q/K/V must share one device")


def _check_centers(key_center, value_center, batch: int, kv_heads: int) -> int:
    # tests/page_gauge_append_extension.cu:765-789; returns the center batch stride
    _require(key_center.is_cuda and value_center.is_cuda, "centers must be CUDA")
    _require(key_center.dtype == torch.float16 and value_center.dtype == torch.float16,
             "centers must be FP16")
    _require(key_center.is_contiguous() and value_center.is_contiguous(),
             "centers must be contiguous")
    shape_ok = key_center.shape == value_center.shape and (
        (batch == 1 and key_center.dim() == 2 and key_center.size(0) == kv_heads
         and key_center.size(1) == HEAD_DIM)
        or (key_center.dim() == 3 and key_center.size(0) == batch
            and key_center.size(1) == kv_heads and key_center.size(2) == HEAD_DIM))
    _require(shape_ok, "centers must be [B,Hkv,128] (or [Hkv,128] for batch one)")
    return 0 if key_center.dim() == 2 else kv_heads * HEAD_DIM


def _check_codes(key_codes, value_codes, key_scales, value_scales, kv_heads: int) -> None:
    _check_tensor(key_codes, "key_codes", torch.int8, 4)
    _check_tensor(value_codes, "value_codes", torch.int8, 4)
    _check_tensor(key_scales, "key_scales", torch.float16, 2)
    _check_tensor(value_scales, "value_scales", torch.float16, 2)
    _require(key_codes.shape == value_codes.shape and key_codes.size(1) == PAGE_SIZE
             and key_codes.size(2) == kv_heads and key_codes.size(3) == HEAD_DIM,
             "INT8 caches must be NHD [pages,16,Hkv,128]")


def _page_gauge_geometry(exact_key_pages, key_codes, key_scales, value_scales, batch: int,
                         kv_heads: int, exact_sink_pages: int) -> tuple[int, int]:
    # tests/page_gauge_append_extension.cu:796-814
    _require(exact_key_pages.size(0) > 0 and exact_key_pages.size(0) % batch == 0
             and key_codes.size(0) % batch == 0,
             "PageGauge pages must be positive and divide evenly across requests")
    exact_pages = exact_key_pages.size(0) // batch
    _require(exact_sink_pages >= 0, "exact prefix page count must be nonnegative")
    _require(exact_pages > exact_sink_pages, "exact cache must retain at least one tail-ring page")
    code_pages = key_codes.size(0) // batch
    _require(exact_sink_pages < code_pages, "exact prefix exceeds the logical cache capacity")
    _require(key_scales.shape == value_scales.shape and key_scales.size(0) == key_codes.size(0)
             and key_scales.size(1) == kv_heads, "scales must be [pages,Hkv]")
    return exact_pages, code_pages


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class PageGaugeAppendExtension:
    """The ``page_gauge_append_ext`` module surface, backed by HIP kernels."""

    def __init__(self) -> None:
        self._lib = _capi.library()

    # -- FP16 append (tests/page_gauge_append_extension.cu:644-745) ---------
    def rope_append_fp16(self, query, key, value, cosine, sine, rotated_query, key_pages,
                         value_pages, position: int) -> None:
        _check_common(query, key, value, cosine, sine, rotated_query, key_pages, value_pages,
                      position)
        _require(position // PAGE_SIZE < key_pages.size(0),
                 "position exceeds the allocated FP16 cache")
        batch = query.size(0)
        _require(key_pages.size(0) % batch == 0,
                 "FP16 cache pages must divide evenly across requests")
        pages_per_request = key_pages.size(0) // batch
        _require(position // PAGE_SIZE < pages_per_request,
                 "position exceeds the per-request FP16 cache capacity")
        _capi.check(self._lib.pg_rope_append_fp16(
            query.data_ptr(), key.data_ptr(), value.data_ptr(), cosine.data_ptr(),
            sine.data_ptr(), rotated_query.data_ptr(), key_pages.data_ptr(),
            value_pages.data_ptr(), query.stride(0), key.stride(0), value.stride(0), batch,
            query.size(1), key.size(1), pages_per_request, int(position), None, 0, 0, _stream()),
            "rope_append_fp16")

    def rope_append_fp16_dynamic(self, query, key, value, cosine, sine, position, rotated_query,
                                 key_pages, value_pages) -> None:
        _check_head_major(query, "query")
        _check_head_major(key, "key")
        _check_head_major(value, "value")
        _check_tensor(rotated_query, "rotated_query", torch.float16, 3)
        _check_tensor(key_pages, "key_pages", torch.float16, 4)
        _check_tensor(value_pages, "value_pages", torch.float16, 4)
        _qkv_checks(query, key, value, rotated_query)
        _require(key_pages.shape == value_pages.shape and key_pages.size(1) == PAGE_SIZE
                 and key_pages.size(2) == key.size(1) and key_pages.size(3) == HEAD_DIM,
                 "page cache must be NHD [pages,16,Hkv,128]")
        _check_dynamic(query, cosine, sine, position)
        batch = query.size(0)
        _require(key_pages.size(0) % batch == 0,
                 "FP16 cache pages must divide evenly across requests")
        _capi.check(self._lib.pg_rope_append_fp16(
            query.data_ptr(), key.data_ptr(), value.data_ptr(), cosine.data_ptr(),
            sine.data_ptr(), rotated_query.data_ptr(), key_pages.data_ptr(),
            value_pages.data_ptr(), query.stride(0), key.stride(0), value.stride(0), batch,
            query.size(1), key.size(1), key_pages.size(0) // batch, 0, position.data_ptr(),
            cosine.stride(0), cosine.size(0), _stream()),
            "rope_append_fp16_dynamic")

    # -- PageGauge append (tests/page_gauge_append_extension.cu:747-948) ----
    def _page_gauge_launch(self, query, key, value, cosine, sine, key_center, value_center,
                           rotated_query, exact_key_pages, exact_value_pages, key_codes,
                           value_codes, key_scales, value_scales, exact_sink_pages: int,
                           host_position: int, device_position, positions, what: str) -> None:
        batch = query.size(0)
        kv_heads = key.size(1)
        center_stride = _check_centers(key_center, value_center, batch, kv_heads)
        _check_codes(key_codes, value_codes, key_scales, value_scales, kv_heads)
        exact_pages, code_pages = _page_gauge_geometry(
            exact_key_pages, key_codes, key_scales, value_scales, batch, kv_heads,
            exact_sink_pages)
        if device_position is None and positions is None:
            _require(host_position // PAGE_SIZE < code_pages,
                     "position exceeds the per-request PageGauge cache capacity")
        ptrs = (query.data_ptr(), key.data_ptr(), value.data_ptr(), cosine.data_ptr(),
                sine.data_ptr())
        tail = (rotated_query.data_ptr(), exact_key_pages.data_ptr(),
                exact_value_pages.data_ptr(), key_codes.data_ptr(), value_codes.data_ptr(),
                key_scales.data_ptr(), value_scales.data_ptr(), query.stride(0), key.stride(0),
                value.stride(0), batch, query.size(1), kv_heads, exact_pages,
                int(exact_sink_pages), code_pages)
        dynamic = device_position is not None or positions is not None
        row_stride = cosine.stride(0) if dynamic else 0
        rows = cosine.size(0) if dynamic else 0
        if positions is not None:
            rc = self._lib.pg_rope_append_page_gauge_positions(
                *ptrs, positions.data_ptr(), key_center.data_ptr(), value_center.data_ptr(),
                center_stride, *tail, row_stride, rows, _stream())
        else:
            rc = self._lib.pg_rope_append_page_gauge(
                *ptrs, key_center.data_ptr(), value_center.data_ptr(), center_stride, *tail,
                int(host_position), None if device_position is None else device_position.data_ptr(),
                row_stride, rows, _stream())
        _capi.check(rc, what)

    def rope_append_page_gauge(self, query, key, value, cosine, sine, key_center, value_center,
                               rotated_query, exact_key_pages, exact_value_pages, key_codes,
                               value_codes, key_scales, value_scales, exact_sink_pages: int,
                               position: int) -> None:
        _check_common(query, key, value, cosine, sine, rotated_query, exact_key_pages,
                      exact_value_pages, position)
        self._page_gauge_launch(query, key, value, cosine, sine, key_center, value_center,
                                rotated_query, exact_key_pages, exact_value_pages, key_codes,
                                value_codes, key_scales, value_scales, exact_sink_pages,
                                position, None, None, "rope_append_page_gauge")

    def _dynamic_head_checks(self, query, key, value, rotated_query, exact_key_pages,
                             exact_value_pages) -> None:
        _check_head_major(query, "query")
        _check_head_major(key, "key")
        _check_head_major(value, "value")
        _check_tensor(rotated_query, "rotated_query", torch.float16, 3)
        _check_tensor(exact_key_pages, "exact_key_pages", torch.float16, 4)
        _check_tensor(exact_value_pages, "exact_value_pages", torch.float16, 4)
        _qkv_checks(query, key, value, rotated_query)
        _require(exact_key_pages.shape == exact_value_pages.shape
                 and exact_key_pages.size(1) == PAGE_SIZE
                 and exact_key_pages.size(2) == key.size(1)
                 and exact_key_pages.size(3) == HEAD_DIM,
                 "exact page cache must be NHD [pages,16,Hkv,128]")

    def rope_append_page_gauge_dynamic(self, query, key, value, cosine, sine, position,
                                       key_center, value_center, rotated_query,
                                       exact_key_pages, exact_value_pages, key_codes,
                                       value_codes, key_scales, value_scales,
                                       exact_sink_pages: int) -> None:
        self._dynamic_head_checks(query, key, value, rotated_query, exact_key_pages,
                                  exact_value_pages)
        _check_dynamic(query, cosine, sine, position)
        self._page_gauge_launch(query, key, value, cosine, sine, key_center, value_center,
                                rotated_query, exact_key_pages, exact_value_pages, key_codes,
                                value_codes, key_scales, value_scales, exact_sink_pages, 0,
                                position, None, "rope_append_page_gauge_dynamic")

    def rope_append_page_gauge_positions(self, query, key, value, cosine, sine, positions,
                                         key_center, value_center, rotated_query,
                                         exact_key_pages, exact_value_pages, key_codes,
                                         value_codes, key_scales, value_scales,
                                         exact_sink_pages: int) -> None:
        """Per-request positions (int32 [B] on the device); RoPE rows are
        taken per request from the [positions,128] tables."""
        self._dynamic_head_checks(query, key, value, rotated_query, exact_key_pages,
                                  exact_value_pages)
        _check_tensor(cosine, "cosine", torch.float16, 2)
        _check_tensor(sine, "sine", torch.float16, 2)
        _check_tensor(positions, "positions", torch.int32, 1)
        _require(cosine.shape == sine.shape and cosine.size(0) > 0 and cosine.size(1) == HEAD_DIM,
                 "dynamic RoPE tables must be matching [positions,128] tensors")
        _require(positions.numel() == query.size(0), "positions must contain one int32 per request")
        self._page_gauge_launch(query, key, value, cosine, sine, key_center, value_center,
                                rotated_query, exact_key_pages, exact_value_pages, key_codes,
                                value_codes, key_scales, value_scales, exact_sink_pages, 0,
                                None, positions, "rope_append_page_gauge_positions")

    def rope_append_page_gauge_slots(self, query, key, value, cosine, sine, positions,
                                     exact_page_ids, code_page_ids, key_center, value_center,
                                     rotated_query, exact_key_pages, exact_value_pages,
                                     key_codes, value_codes, key_scales, value_scales) -> None:
        """Per-request positions with explicit exact and code page ids (device
        int32 [B] each), as a serving block table gives them; centers are
        per row ([B,Hkv,128], or [Hkv,128] for batch one)."""
        self._dynamic_head_checks(query, key, value, rotated_query, exact_key_pages,
                                  exact_value_pages)
        _check_tensor(cosine, "cosine", torch.float16, 2)
        _check_tensor(sine, "sine", torch.float16, 2)
        _require(cosine.shape == sine.shape and cosine.size(0) > 0 and cosine.size(1) == HEAD_DIM,
                 "dynamic RoPE tables must be matching [positions,128] tensors")
        batch = query.size(0)
        for tensor, name in ((positions, "positions"), (exact_page_ids, "exact_page_ids"),
                             (code_page_ids, "code_page_ids")):
            _check_tensor(tensor, name, torch.int32, 1)
            _require(tensor.numel() == batch, f"{name} must contain one int32 per request")
        kv_heads = key.size(1)
        center_stride = _check_centers(key_center, value_center, batch, kv_heads)
        _check_codes(key_codes, value_codes, key_scales, value_scales, kv_heads)
        _require(key_scales.shape == value_scales.shape and key_scales.size(0) == key_codes.size(0)
                 and key_scales.size(1) == kv_heads, "scales must be [pages,Hkv]")
        _capi.check(self._lib.pg_rope_append_page_gauge_slots(
            query.data_ptr(), key.data_ptr(), value.data_ptr(), cosine.data_ptr(),
            sine.data_ptr(), positions.data_ptr(), exact_page_ids.data_ptr(),
            code_page_ids.data_ptr(), key_center.data_ptr(), value_center.data_ptr(),
            center_stride, rotated_query.data_ptr(), exact_key_pages.data_ptr(),
            exact_value_pages.data_ptr(), key_codes.data_ptr(), value_codes.data_ptr(),
            key_scales.data_ptr(), value_scales.data_ptr(), query.stride(0), key.stride(0),
            value.stride(0), batch, query.size(1), kv_heads, exact_key_pages.size(0),
            key_codes.size(0), cosine.stride(0), cosine.size(0), _stream()),
            "rope_append_page_gauge_slots")

    # -- fused exact tail (tests/page_gauge_append_extension.cu:950-1028) ---
    def exact_tail_merge_center(self, query, exact_key_pages, exact_value_pages,
                                exact_page_indices, exact_last_page_len, old_output, old_lse,
                                value_center, sm_scale: float) -> None:
        _check_tensor(query, "query", torch.float16, 3)
        _check_tensor(exact_key_pages, "exact_key_pages", torch.float16, 4)
        _check_tensor(exact_value_pages, "exact_value_pages", torch.float16, 4)
        _check_tensor(exact_page_indices, "exact_page_indices", torch.int32, 1)
        _check_tensor(exact_last_page_len, "exact_last_page_len", torch.int32, 1)
        _check_tensor(old_output, "old_output", torch.float16, 3)
        _check_tensor(old_lse, "old_lse", torch.float32, 2)
        _require(value_center.is_cuda and value_center.dtype == torch.float16
                 and value_center.is_contiguous(), "value_center must be contiguous CUDA FP16")
        _require(query.shape == old_output.shape, "query and old output shapes must match")
        _require(query.size(2) == HEAD_DIM, "head dimension must be 128")
        _require(exact_key_pages.shape == exact_value_pages.shape
                 and exact_key_pages.size(1) == PAGE_SIZE and exact_key_pages.size(3) == HEAD_DIM,
                 "exact caches must be matching NHD [pages,16,Hkv,128] tensors")
        query_heads = query.size(1)
        batch = query.size(0)
        _require(batch > 0, "batch size must be positive")
        kv_heads = exact_key_pages.size(2)
        _require(query_heads > 0 and kv_heads > 0 and query_heads % kv_heads == 0,
                 "query heads must be a positive multiple of KV heads")
        _require(query_heads // kv_heads == 4,
                 "the fused exact-tail kernel currently requires GQA group size 4")
        _require(old_lse.size(0) == batch and old_lse.size(1) == query_heads,
                 "old_lse must be [B,Hq]")
        center_ok = ((batch == 1 and value_center.dim() == 2 and value_center.size(0) == kv_heads
                      and value_center.size(1) == HEAD_DIM)
                     or (value_center.dim() == 3 and value_center.size(0) == batch
                         and value_center.size(1) == kv_heads and value_center.size(2) == HEAD_DIM))
        _require(center_ok, "value_center must be [B,Hkv,128] (or [Hkv,128] for batch one)")
        _require(exact_last_page_len.numel() == batch,
                 "exact_last_page_len must contain one device scalar per request")
        _require(exact_page_indices.numel() % batch == 0,
                 "exact page indices must divide evenly across requests")
        pages = exact_page_indices.numel() // batch
        _require(0 < pages <= 16, "the fused exact tail supports 1..16 pages per request")
        _require(exact_key_pages.size(0) >= batch * pages,
                 "exact page index count exceeds the ring allocation")
        _require(sm_scale > 0.0 and sm_scale != float("inf"), "sm_scale must be positive and finite")
        center_stride = 0 if value_center.dim() == 2 else kv_heads * HEAD_DIM
        _capi.check(self._lib.pg_exact_tail_merge_center(
            query.data_ptr(), exact_key_pages.data_ptr(), exact_value_pages.data_ptr(),
            exact_page_indices.data_ptr(), exact_last_page_len.data_ptr(), old_output.data_ptr(),
            old_lse.data_ptr(), value_center.data_ptr(), center_stride, batch, query_heads,
            kv_heads, pages, float(sm_scale), _stream()),
            "exact_tail_merge_center")


_EXTENSION: PageGaugeAppendExtension | None = None


def load_append_extension() -> PageGaugeAppendExtension:
    """Return the append extension (scripts/page_gauge_runtime.py:16-29).

    Raises ``RuntimeError`` without a GPU, like the reference loader, and
    ``LibraryMissingError`` if ``libpagegauge_hip.so`` was not built.
    """
    global _EXTENSION
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required for the PageGauge append extension")
    if _EXTENSION is None:
        _EXTENSION = PageGaugeAppendExtension()
    return _EXTENSION
