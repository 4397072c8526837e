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


def quantize_page_gauge(values: torch.Tensor, center: torch.Tensor | None = None):
    """The K1 driver's quantizer (scripts/benchmark_flashinfer_page_affine_int8.py:256-278).

    ``values`` [pages, 16, H, 128] fp16 on the GPU.  Returns ``(codes, center,
    scale, reconstructed_centered, centered)`` like the reference:
    * center: the per-(head, dim) mean over every page and token, as FP16
      (``token_major_centers``: the exact mean; the reference's float32
      ``mean`` agrees except where its own rounding crosses a half-ulp
      boundary), unless given;
    * codes and scale from ``pg_quantize_page_gauge``: float32-centered values,
      scale fp16(max(amax/127, 2^-20)) per (page, head), round-half-even codes;
    * reconstructed_centered = fp16(codes * scale), centered = fp16(values -
      center) (element-wise, as the reference returns them).
    """
    if values.ndim != 4 or values.shape[1] != PAGE or values.shape[3] != DIM:
        raise ValueError("values must be [pages, 16, HKV, 128]")
    if values.dtype != torch.float16:
        raise ValueError("values must be float16")
    pages, heads = int(values.shape[0]), int(values.shape[2])
    if center is None:
        flat = values.view(pages * PAGE, heads, DIM)
        center = token_major_centers(flat, flat)[0]
    if tuple(center.shape) != (heads, DIM) or center.dtype != torch.float16:
        raise ValueError("center must be float16 [heads, 128]")
    _all_cuda_contiguous(values, center)
    codes = torch.empty(values.shape, dtype=torch.int8, device=values.device)
    scale = torch.empty(pages, heads, dtype=torch.float16, device=values.device)
    _capi.call("pg_quantize_page_gauge", values.data_ptr(), center.data_ptr(), codes.data_ptr(),
               scale.data_ptr(), pages, heads, _stream())
    reconstructed = (codes.float() * scale.float()[:, None, :, None]).half()
    centered = (values.float() - center.float()[None, None]).half()
    return codes, center, scale, reconstructed, centered


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


def _token_rows(t: torch.Tensor) -> int:
    """Token stride (elements) of a [T, H, 128] FP16 tensor whose (H, 128) rows are dense."""
    if not t.is_cuda or t.dtype != torch.float16:
        raise ValueError("token-major K/V must be CUDA float16")
    if t.stride(2) != 1 or t.stride(1) != DIM or t.stride(0) < t.shape[1] * DIM or t.stride(0) % 2:
        raise ValueError("token-major K/V rows must be dense [heads,128] blocks")
    return t.stride(0)


def token_major_centers(source_key: torch.Tensor, source_value: torch.Tensor,
                        key_center: torch.Tensor | None = None,
                        value_center: torch.Tensor | None = None,
                        workspace: torch.Tensor | None = None):
    """Per-(head, dim) token means of token-major [T,Hkv,128] K/V, as FP16.

    HIP replacement of ``token_major_centers``
    (diagnostics/benchmark_backend_exclusive.py:372-395), same shape checks and
    messages.  The sum is exact (int64 multiples of 2^-24), so the result is
    f16(f32(exact_sum / T)) whatever the reduction order.  Token rows may be
    strided (a K or V slice of a fused QKV projection).  Outputs may be given
    (e.g. ``cache.key_center[layer, request]``); ``workspace`` is a uint8 CUDA
    tensor of at least ``pg_token_major_centers_workspace_bytes`` bytes.
    """
    if source_key.shape != source_value.shape or source_key.ndim != 3:
        raise ValueError("token-major K/V must have identical [T,Hkv,D] shapes")
    if source_key.shape[0] <= 0 or source_key.shape[1] <= 0:
        raise ValueError("token-major K/V must contain tokens and heads")
    if int(source_key.shape[2]) != DIM:
        raise ValueError(f"token-major K/V head dimension must be {DIM}")
    tokens, heads = int(source_key.shape[0]), int(source_key.shape[1])
    key_stride, value_stride = _token_rows(source_key), _token_rows(source_value)
    shape = (heads, DIM)
    if key_center is None:
        key_center = torch.empty(shape, device=source_key.device, dtype=torch.float16)
    if value_center is None:
        value_center = torch.empty(shape, device=source_key.device, dtype=torch.float16)
    for center in (key_center, value_center):
        if tuple(center.shape) != shape or center.dtype != torch.float16:
            raise ValueError(f"centers must be float16 {shape}")
    _all_cuda_contiguous(key_center, value_center)
    lib = _capi.library()
    need = int(lib.pg_token_major_centers_workspace_bytes(tokens, heads))
    if workspace is None:
        workspace = torch.empty(need, device=source_key.device, dtype=torch.uint8)
    if workspace.dtype != torch.uint8 or workspace.numel() < need:
        raise ValueError(f"center workspace must be a uint8 tensor of at least {need} bytes")
    _all_cuda_contiguous(workspace)
    _capi.call("pg_token_major_centers", source_key.data_ptr(), key_stride,
               source_value.data_ptr(), value_stride, tokens, heads, key_center.data_ptr(),
               value_center.data_ptr(), workspace.data_ptr(), workspace.numel(), _stream())
    return key_center, value_center


def prefill_page_gauge(source_key: torch.Tensor, source_value: torch.Tensor,
                       key_center: torch.Tensor, value_center: torch.Tensor,
                       key_codes: torch.Tensor, value_codes: torch.Tensor,
                       key_scales: torch.Tensor, value_scales: torch.Tensor,
                       exact_page_map: torch.Tensor | None = None,
                       exact_key_pages: torch.Tensor | None = None,
                       exact_value_pages: torch.Tensor | None = None) -> None:
    """Quantise a token-major prefix into INT8 pages and store its exact pages.

    Mirrors the cache population of ``populate_backend_cache_layer``
    (diagnostics/benchmark_backend_exclusive.py:442-506): every page gets
    codes and scales from float32-centered values (``quantize_completed_kv_pages``
    arithmetic) and page ``i`` with ``exact_page_map[i] >= 0`` is also written
    as ``fp16(f32(x) - f32(center))`` into that ring page.  ``source_*`` are
    [pages*16, Hkv, 128] FP16 (token rows may be strided).
    """
    if source_key.shape != source_value.shape or source_key.ndim != 3:
        raise ValueError("token-major K/V must have identical [T,Hkv,D] shapes")
    tokens, heads = int(source_key.shape[0]), int(source_key.shape[1])
    if tokens <= 0 or tokens % PAGE or int(source_key.shape[2]) != DIM:
        raise ValueError("prefill K/V must be whole 16-token pages of [Hkv,128] rows")
    pages = tokens // PAGE
    key_stride, value_stride = _token_rows(source_key), _token_rows(source_value)
    if key_center.shape != (heads, DIM) or value_center.shape != key_center.shape:
        raise ValueError("centers must be [heads, 128]")
    for codes in (key_codes, value_codes):
        if codes.dtype != torch.int8 or tuple(codes.shape) != (pages, PAGE, heads, DIM):
            raise ValueError("codes must be int8 [pages,16,heads,128]")
    for scales in (key_scales, value_scales):
        if scales.dtype != torch.float16 or tuple(scales.shape) != (pages, heads):
            raise ValueError("scales must be float16 [pages,heads]")
    _all_cuda_contiguous(key_center, value_center, key_codes, value_codes, key_scales,
                         value_scales)
    map_ptr = ring_k = ring_v = None
    if exact_page_map is not None:
        if exact_page_map.dtype != torch.int32 or tuple(exact_page_map.shape) != (pages,):
            raise ValueError("exact_page_map must be int32 [pages]")
        if exact_key_pages is None or exact_value_pages is None:
            raise ValueError("an exact page map needs exact key/value pages")
        for ring in (exact_key_pages, exact_value_pages):
            if ring.dtype != torch.float16 or ring.ndim != 4 or tuple(ring.shape[1:]) != (PAGE, heads, DIM):
                raise ValueError("exact pages must be float16 [ring_pages,16,heads,128]")
        _all_cuda_contiguous(exact_page_map, exact_key_pages, exact_value_pages)
        valid = exact_page_map[exact_page_map >= 0]
        if valid.numel() and int(valid.max()) >= exact_key_pages.shape[0]:
            raise ValueError("exact_page_map points past the exact pages")
        map_ptr = exact_page_map.data_ptr()
        ring_k, ring_v = exact_key_pages.data_ptr(), exact_value_pages.data_ptr()
    _capi.call("pg_prefill_page_gauge", source_key.data_ptr(), key_stride, source_value.data_ptr(),
               value_stride, key_center.data_ptr(), value_center.data_ptr(), key_codes.data_ptr(),
               value_codes.data_ptr(), key_scales.data_ptr(), value_scales.data_ptr(), map_ptr,
               ring_k, ring_v, pages, heads, _stream())
