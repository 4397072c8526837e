"""Paged-decode operators with the reference's wrapper call shapes.

The reference drives a patched FlashInfer ``BatchDecodeWithPagedKVCacheWrapper``
(``scripts/benchmark_flashinfer_page_affine_int8.py:192-231``, ``:363-389``,
``:566-602``) and ``flashinfer.merge_state_in_place``.  This module offers the
same ``plan``/``run`` surface on top of ``libpagegauge_hip.so``:

* ``BatchDecodeWithPagedKVCacheWrapper`` -- FP16 pages, or INT8 page-affine
  PageGauge pages when planned with ``kv_data_type=torch.int8`` (then ``run``
  takes ``k_page_scale, v_page_scale, sm_scale`` like the JIT variant);
* ``make_page_gauge_wrapper`` -- the INT8 factory of the reference;
* ``PageGaugeSegmentedDecode`` -- INT8 history + FP16 exact tail + value
  center in one planned call (the reference's four-launch ``run_affine``);
* ``merge_state_in_place`` and ``segment_page_table``.

Everything runs on the current HIP stream and never synchronises in ``run``.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Sequence

import torch

from . import _capi

HQ = 32
HKV = 8
DIM = 128
PAGE = 16


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _num_cus(device: torch.device) -> int:
    try:
        return int(torch.cuda.get_device_properties(device).multi_processor_count)
    except Exception:  # pragma: no cover - property unavailable
        return 256


def _host_i32(tensor: torch.Tensor | Sequence[int]) -> torch.Tensor:
    if isinstance(tensor, torch.Tensor):
        return tensor.detach().to("cpu", torch.int32).contiguous()
    return torch.tensor(list(tensor), dtype=torch.int32)


def _ptr(tensor: Optional[torch.Tensor]):
    return None if tensor is None else tensor.data_ptr()


def _host_tables(indptr, last_page_len, indices: Optional[torch.Tensor] = None,
                 what: str = "") -> tuple[torch.Tensor, torch.Tensor]:
    """Host int32 copies of a CSR page table's ``indptr`` and
    ``last_page_len``, checked against each other and against ``indices``
    (its length only) before the planner reads them: the planner reads
    ``last_page_len[b]`` for every request and the kernels read
    ``indices[indptr[0]:indptr[B]]``, so a short tensor would be read past
    its end."""
    prefix = f"{what} " if what else ""
    host_indptr = _host_i32(indptr)
    host_last = _host_i32(last_page_len)
    if host_indptr.dim() != 1 or host_indptr.numel() < 2:
        raise ValueError(f"{prefix}indptr must be a 1-D tensor of batch_size + 1 >= 2 entries")
    batch = host_indptr.numel() - 1
    if host_last.dim() != 1 or host_last.numel() != batch:
        raise ValueError(f"{prefix}last_page_len must have one entry per request "
                         f"({batch}), got {host_last.numel()}")
    if int(host_indptr[0]) < 0:
        raise ValueError(f"{prefix}indptr[0] must be non-negative")
    if batch > 0 and bool((host_indptr[1:] < host_indptr[:-1]).any()):
        raise ValueError(f"{prefix}indptr must be non-decreasing")
    if indices is not None and indices.numel() < int(host_indptr[-1]):
        raise ValueError(f"{prefix}indices has {indices.numel()} entries but indptr[-1] is "
                         f"{int(host_indptr[-1])}")
    return host_indptr, host_last


# Opt-in page-id bounds check (debug builds of a caller): with
# PAGEGAUGE_CHECK_PAGE_IDS=1 in the environment (or ``CHECK_PAGE_IDS = True``
# set on this module), ``plan()`` copies the planned page ids to the host and
# every ``run()`` / ``bind()`` verifies that they index the pools it is given.
# The kernels themselves trust the tables, as the reference's do.
CHECK_PAGE_IDS = os.environ.get("PAGEGAUGE_CHECK_PAGE_IDS", "0") not in ("", "0")


def _page_id_range(indices: torch.Tensor, host_indptr: torch.Tensor):
    """(min, max) of the planned ids ``indices[indptr[0]:indptr[-1]]``, or
    None when the check is off or the table is empty."""
    if not CHECK_PAGE_IDS:
        return None
    lo, hi = int(host_indptr[0]), int(host_indptr[-1])
    if hi <= lo:
        return None
    ids = indices[lo:hi].detach().to("cpu")
    return int(ids.min()), int(ids.max())


def _check_page_ids(id_range, pool_pages: int, what: str) -> None:
    if id_range is not None and (id_range[0] < 0 or id_range[1] >= pool_pages):
        raise ValueError(f"{what} page ids span [{id_range[0]}, {id_range[1]}] but the pool "
                         f"holds {pool_pages} pages")


def _check_query(q: torch.Tensor, batch: int, num_qo_heads: int) -> None:
    if not q.is_cuda or q.dtype != torch.float16 or q.dim() != 3:
        raise ValueError("q must be a CUDA float16 [B, Hq, 128] tensor")
    if tuple(q.shape) != (batch, num_qo_heads, DIM):
        raise ValueError(f"q shape {tuple(q.shape)} does not match the plan ({batch},{num_qo_heads},{DIM})")
    if q.stride(2) != 1 or q.stride(1) != DIM or q.stride(0) % 8 or q.data_ptr() % 16:
        raise ValueError("q rows must be contiguous and 16-byte aligned")


def _check_cache(cache: torch.Tensor, name: str, dtype: torch.dtype, num_kv_heads: int) -> None:
    if not cache.is_cuda or cache.dtype != dtype or cache.dim() != 4 or not cache.is_contiguous():
        raise ValueError(f"{name} must be a contiguous CUDA {dtype} [pages,16,Hkv,128] tensor")
    if tuple(cache.shape[1:]) != (PAGE, num_kv_heads, DIM):
        raise ValueError(f"{name} must be NHD [pages,16,{num_kv_heads},128]")


def _check_scale(scale: torch.Tensor, name: str, pages: int, num_kv_heads: int) -> None:
    if (not scale.is_cuda or scale.dtype != torch.float16 or not scale.is_contiguous()
            or tuple(scale.shape) != (pages, num_kv_heads)):
        raise ValueError(f"{name} must be a contiguous CUDA float16 [{pages},{num_kv_heads}] tensor")


def _check_index(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda or t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous CUDA int32 tensor")


def _finalize_args(finalize, batch: int, code_pages: int):
    """(positions, position stride, code pages per request) of a finalize."""
    positions, per_request = finalize
    _check_index(positions, "finalize positions")
    if positions.numel() not in (1, batch):
        raise ValueError("finalize positions must be one per request or one shared")
    per_request = int(per_request)
    if per_request <= 0 or per_request * batch > code_pages:
        raise ValueError("code pages per request exceed the code pool")
    return positions, (1 if positions.numel() == batch and batch > 1 else 0), per_request


class _Planned:
    """Holds a C plan, the device index tensors it refers to and the workspace."""

    def __init__(self, workspace: torch.Tensor) -> None:
        if not workspace.is_cuda or workspace.dtype != torch.uint8 or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous CUDA uint8 tensor")
        self.workspace = workspace
        self.plan = _capi.DecodePlan()
        self.planned = False
        self.generation = 0     # advances with every plan written into ``self.plan``

    def make_plan(self, host_indptr, host_last, primary_kind, host_tail_indptr, host_tail_last,
                  num_qo_heads, num_kv_heads, head_dim, page_size, split_pages, tail_split_pages,
                  device, num_cus: Optional[int] = None, exact_tail_pages_hint: int = 0) -> None:
        lib = _capi.library()
        batch = host_indptr.numel() - 1
        rc = lib.pg_decode_plan(
            host_indptr.data_ptr(), host_last.data_ptr(), batch, primary_kind,
            None if host_tail_indptr is None else host_tail_indptr.data_ptr(),
            None if host_tail_last is None else host_tail_last.data_ptr(),
            num_qo_heads, num_kv_heads, head_dim, page_size, int(split_pages or 0),
            int(tail_split_pages or 0), int(exact_tail_pages_hint), int(num_cus or _num_cus(device)),
            self.workspace.data_ptr(), self.workspace.numel(), ctypes.byref(self.plan), _stream())
        _capi.check(rc, "decode plan")
        self.planned = True
        self.generation += 1

    @property
    def split_pages(self) -> int:
        return int(self.plan.split_pages)

    @property
    def num_items(self) -> int:
        return int(self.plan.num_items)


WORK_ITEM_FIELDS = ("request", "kind", "segment", "page_begin", "page_end", "last_page",
                    "item_in_request", "items_in_request", "request_page_begin", "page_weight",
                    "reserved0", "reserved1")


def plan_work_items(indptr, last_page_len, tail_indptr=None, tail_last_page_len=None,
                    kv_data_type=torch.int8, num_qo_heads: int = HQ, num_kv_heads: int = HKV,
                    head_dim: int = DIM, page_size: int = PAGE, split_pages: int = 0,
                    tail_split_pages: int = 0, num_cus: int = 256, exact_tail_pages_hint: int = 0):
    """Run the decode scheduler on the host only (no device, no workspace).

    Returns ``(plan, items, item_ptr)``: the ``DecodePlan`` that
    ``pg_decode_plan`` would produce, the work list as an int32 tensor
    [num_items, 12] with columns ``WORK_ITEM_FIELDS``, and [B+1] per-request
    item offsets.  Same validation and error messages as ``plan``.
    """
    lib = _capi.library()
    host_indptr, host_last = _host_tables(indptr, last_page_len)
    host_tail = host_tail_last = None
    if (tail_indptr is None) != (tail_last_page_len is None):
        raise ValueError("tail indptr and last_page_len go together")
    if tail_indptr is not None:
        host_tail, host_tail_last = _host_tables(tail_indptr, tail_last_page_len, what="tail")
        if host_tail.numel() != host_indptr.numel():
            raise ValueError("old and tail page tables must cover the same batch")
    batch = host_indptr.numel() - 1
    kind = {torch.int8: _capi.PG_KV_INT8, torch.float16: _capi.PG_KV_FP16,
            "heterogeneous": _capi.PG_KV_HETEROGENEOUS}[kv_data_type]
    plan = _capi.DecodePlan()
    args = (host_indptr.data_ptr(), host_last.data_ptr(), batch, kind,
            None if host_tail is None else host_tail.data_ptr(),
            None if host_tail_last is None else host_tail_last.data_ptr(), num_qo_heads,
            num_kv_heads, head_dim, page_size, int(split_pages), int(tail_split_pages),
            int(exact_tail_pages_hint), int(num_cus), ctypes.byref(plan))
    _capi.check(lib.pg_decode_plan_host(*args, None, 0, None), "decode plan")
    items = torch.empty(max(1, plan.num_items), len(WORK_ITEM_FIELDS), dtype=torch.int32)
    item_ptr = torch.empty(batch + 1, dtype=torch.int32)
    _capi.check(lib.pg_decode_plan_host(*args, items.data_ptr(), items.size(0),
                                        item_ptr.data_ptr()), "decode plan")
    return plan, items[:plan.num_items], item_ptr


class BoundDecode:
    """A planned decode with every pointer resolved, for serving loops and
    timing: ``__call__`` issues the call (``pg_decode_run``: the partial and
    the combine kernels), ``partial()`` / ``combine()`` the two kernels
    separately, and ``timed(start, stop)`` the call with two timing events
    stamped by its first and last kernel dispatches.  No tensor validation
    happens here; the object holds references to the tensors it was bound to
    (their storage must not be resized or swapped), and it is valid until its
    wrapper plans again: a call after a new ``plan()`` raises RuntimeError,
    since the plan and workspace then describe other tables.  ``stream`` is a
    raw hipStream_t handle (default: the current stream when ``bind`` was
    called)."""

    def __init__(self, state: "_Planned", partial_args: tuple, combine_args: tuple,
                 stream: int, keep: tuple = ()) -> None:
        lib = _capi.library()
        self._state = state
        self._generation = state.generation
        self._keep = keep
        self._plan_ref = ctypes.byref(state.plan)
        self._partial = lib.pg_decode_run_partial
        self._partial_timed = lib.pg_decode_run_partial_timed
        self._combine = lib.pg_decode_run_combine
        self._run = lib.pg_decode_run
        self._run_timed = lib.pg_decode_run_timed
        ws = state.workspace.data_ptr()
        self._partial_args = (self._plan_ref, *partial_args, ws, stream)
        self._combine_args = (self._plan_ref, *combine_args, ws, stream)
        # pg_decode_run: partial inputs (without sm_scale), combine outputs, sm_scale
        self._run_args = (self._plan_ref, *partial_args[:-1], *combine_args, partial_args[-1], ws,
                          stream)

    def _check_plan(self) -> None:
        if self._state.generation != self._generation:
            raise RuntimeError("the decode was planned again after bind(); bind it again")

    def partial(self) -> None:
        self._check_plan()
        rc = self._partial(*self._partial_args)
        if rc:
            _capi.check(rc, "decode partial")

    def partial_timed(self, start_event: int, stop_event: int) -> None:
        """``partial()`` whose kernel dispatch itself stamps two timing events
        (raw hipEvent_t handles, e.g. ``torch.cuda.Event(enable_timing=True)``
        ``.cuda_event`` after one ``record()``): their elapsed time is the
        kernel's duration without the launch gap."""
        self._check_plan()
        rc = self._partial_timed(*self._partial_args, start_event, stop_event)
        if rc:
            _capi.check(rc, "decode partial")

    def combine(self) -> None:
        self._check_plan()
        rc = self._combine(*self._combine_args)
        if rc:
            _capi.check(rc, "decode combine")

    def timed(self, start_event: int, stop_event: int) -> None:
        self._check_plan()
        rc = self._run_timed(*self._run_args, start_event, stop_event)
        if rc:
            _capi.check(rc, "decode run")

    def __call__(self) -> None:
        self._check_plan()
        rc = self._run(*self._run_args)
        if rc:
            _capi.check(rc, "decode run")


class BatchDecodeWithPagedKVCacheWrapper:
    """FlashInfer-shaped paged decode over FP16 or PageGauge INT8 pages.

    ``plan(indptr, indices, last_page_len, num_qo_heads, num_kv_heads,
    head_dim, page_size, pos_encoding_mode="NONE", q_data_type=fp16,
    kv_data_type=fp16|int8, o_data_type=fp16, sm_scale=None,
    fixed_split_size=None)`` as called by
    scripts/benchmark_flashinfer_page_affine_int8.py:363-389.  ``indices`` and
    ``last_page_len`` must stay alive (and may be updated in place) until the
    next ``plan``; ``last_page_len`` is re-read by every ``run``.
    """

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, use_tensor_cores: bool = True,
                 backend: str = "auto", **_unused) -> None:
        if kv_layout != "NHD":
            raise ValueError("only the NHD layout is supported")
        self._state = _Planned(float_workspace_buffer)
        self._kv_dtype = None
        self._sm_scale = None
        self.use_cuda_graph = use_cuda_graph

    def plan(self, indptr, indices, last_page_len, num_qo_heads: int, num_kv_heads: int,
             head_dim: int, page_size: int, pos_encoding_mode: str = "NONE",
             window_left: int = -1, logits_soft_cap=None, q_data_type=torch.float16,
             kv_data_type=None, o_data_type=None, data_type=None, sm_scale=None,
             rope_scale=None, rope_theta=None, non_blocking: bool = True,
             fixed_split_size: Optional[int] = None, disable_split_kv: bool = False,
             num_cus: Optional[int] = None, **_unused) -> None:
        if pos_encoding_mode != "NONE":
            raise ValueError("only pos_encoding_mode='NONE' is supported")
        if window_left not in (-1, None) or logits_soft_cap not in (None, 0.0):
            raise ValueError("sliding windows and logit soft caps are not supported")
        kv_dtype = kv_data_type if kv_data_type is not None else (data_type or torch.float16)
        if q_data_type not in (torch.float16, None) or kv_dtype not in (torch.float16, torch.int8):
            raise ValueError("q must be float16 and KV float16 or int8")
        if o_data_type not in (None, torch.float16):
            raise ValueError("output must be float16")
        _check_index(indices, "indices")
        _check_index(last_page_len, "last_page_len")
        host_indptr, host_last = _host_tables(indptr, last_page_len, indices)
        kind = _capi.PG_KV_INT8 if kv_dtype == torch.int8 else _capi.PG_KV_FP16
        split = 1 << 30 if disable_split_kv else (fixed_split_size or 0)
        self._state.make_plan(host_indptr, host_last, kind, None, None, num_qo_heads, num_kv_heads,
                              head_dim, page_size, split, 0, indices.device, num_cus)
        self._indices = indices
        self._last_page_len = last_page_len
        self._id_range = _page_id_range(indices, host_indptr)
        self._kv_dtype = kv_dtype
        self._batch = host_indptr.numel() - 1
        self._num_qo_heads = num_qo_heads
        self._num_kv_heads = num_kv_heads
        self._sm_scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(head_dim)

    @property
    def split_pages(self) -> int:
        return self._state.split_pages

    @property
    def num_work_items(self) -> int:
        return self._state.num_items

    def run(self, q: torch.Tensor, paged_kv_cache, *args, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None, return_lse: bool = False, **_unused):
        if not self._state.planned:
            raise RuntimeError("plan() must be called before run()")
        k_cache, v_cache = paged_kv_cache
        _check_query(q, self._batch, self._num_qo_heads)
        k_scale = v_scale = None
        sm_scale = self._sm_scale
        if self._kv_dtype == torch.int8:
            if len(args) < 2:
                raise ValueError("INT8 PageGauge run needs k_page_scale and v_page_scale")
            k_scale, v_scale = args[0], args[1]
            if len(args) > 2:
                sm_scale = float(args[2])
            _check_cache(k_cache, "k_cache", torch.int8, self._num_kv_heads)
            _check_cache(v_cache, "v_cache", torch.int8, self._num_kv_heads)
            _check_scale(k_scale, "k_page_scale", k_cache.size(0), self._num_kv_heads)
            _check_scale(v_scale, "v_page_scale", v_cache.size(0), self._num_kv_heads)
        else:
            _check_cache(k_cache, "k_cache", torch.float16, self._num_kv_heads)
            _check_cache(v_cache, "v_cache", torch.float16, self._num_kv_heads)
        _check_page_ids(self._id_range, min(k_cache.size(0), v_cache.size(0)), "KV")
        if out is None:
            out = torch.empty_like(q)
        if return_lse and lse is None:
            lse = torch.empty(q.size(0), q.size(1), device=q.device, dtype=torch.float32)
        _capi.call("pg_decode_run", ctypes.byref(self._state.plan), q.data_ptr(), q.stride(0),
                   k_cache.data_ptr(), v_cache.data_ptr(), _ptr(k_scale), _ptr(v_scale),
                   self._indices.data_ptr(), self._last_page_len.data_ptr(), None, None, None,
                   None, None, 0, out.data_ptr(), _ptr(lse), float(sm_scale),
                   self._state.workspace.data_ptr(), _stream())
        return (out, lse) if return_lse else out

    def bind(self, q, paged_kv_cache, k_page_scale=None, v_page_scale=None, sm_scale=None,
             out=None, lse=None, stream: Optional[int] = None) -> BoundDecode:
        """Resolve a ``run`` once; see ``BoundDecode``."""
        if not self._state.planned:
            raise RuntimeError("plan() must be called before bind()")
        if out is None:
            raise ValueError("bind needs a preallocated out tensor")
        args = () if self._kv_dtype != torch.int8 else (k_page_scale, v_page_scale)
        self.run(q, paged_kv_cache, *args, out=out, lse=lse)   # validates once
        k_cache, v_cache = paged_kv_cache
        scale = self._sm_scale if sm_scale is None else sm_scale
        partial = (q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
                   _ptr(k_page_scale), _ptr(v_page_scale), self._indices.data_ptr(),
                   self._last_page_len.data_ptr(), None, None, None, None, float(scale))
        combine = (None, 0, out.data_ptr(), _ptr(lse))
        keep = (q, k_cache, v_cache, k_page_scale, v_page_scale, self._indices,
                self._last_page_len, out, lse)
        return BoundDecode(self._state, partial, combine, _stream() if stream is None else stream,
                           keep)


def make_page_gauge_wrapper(flashinfer_module, workspace: torch.Tensor, **wrapper_kwargs):
    """INT8 PageGauge wrapper (scripts/benchmark_flashinfer_page_affine_int8.py:192-231).

    The first argument (the flashinfer module in the reference) is ignored.
    """
    wrapper = BatchDecodeWithPagedKVCacheWrapper(workspace, "NHD", **wrapper_kwargs)
    wrapper.page_gauge_module_uri = "pagegauge_amd/libpagegauge_hip.so"
    return wrapper


class PageGaugeSegmentedDecode:
    """INT8 history pages + FP16 exact tail + value center in one plan/run.

    Equivalent to the reference's ``run_affine``
    (scripts/benchmark_flashinfer_page_affine_int8.py:566-602): INT8 decode
    with page scales, FP16 tail decode, ``merge_state_in_place`` and
    ``add_(output_center)`` -- here a single partial kernel covering both
    segments plus one combine kernel.
    """

    def __init__(self, workspace: torch.Tensor) -> None:
        self._state = _Planned(workspace)

    def plan(self, old_indptr, old_indices, old_last_page_len, tail_indptr, tail_indices,
             tail_last_page_len, num_qo_heads: int = HQ, num_kv_heads: int = HKV,
             head_dim: int = DIM, page_size: int = PAGE, sm_scale: Optional[float] = None,
             fixed_split_size: Optional[int] = None,
             tail_split_size: Optional[int] = None, num_cus: Optional[int] = None) -> None:
        """``num_cus``: workgroups the balanced plan targets (default: the
        device's CU count)."""
        for t, n in ((old_indices, "old_indices"), (old_last_page_len, "old_last_page_len"),
                     (tail_indices, "tail_indices"), (tail_last_page_len, "tail_last_page_len")):
            _check_index(t, n)
        host_old, host_old_last = _host_tables(old_indptr, old_last_page_len, old_indices, "old")
        host_tail, host_tail_last = _host_tables(tail_indptr, tail_last_page_len, tail_indices,
                                                 "tail")
        if host_old.numel() != host_tail.numel():
            raise ValueError("old and tail page tables must cover the same batch")
        self._state.make_plan(host_old, host_old_last, _capi.PG_KV_INT8, host_tail,
                              host_tail_last, num_qo_heads, num_kv_heads, head_dim,
                              page_size, fixed_split_size or 0, tail_split_size or 0,
                              old_indices.device, num_cus)
        self._old = (old_indices, old_last_page_len)
        self._tail = (tail_indices, tail_last_page_len)
        self._id_ranges = (_page_id_range(old_indices, host_old),
                           _page_id_range(tail_indices, host_tail))
        self._batch = host_old.numel() - 1
        self._num_qo_heads = num_qo_heads
        self._num_kv_heads = num_kv_heads
        self._sm_scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(head_dim)

    @property
    def split_pages(self) -> int:
        return self._state.split_pages

    @property
    def tail_split_pages(self) -> int:
        return int(self._state.plan.tail_split_pages)

    @property
    def num_work_items(self) -> int:
        return self._state.num_items

    def run(self, q, codes, k_page_scale, v_page_scale, exact_cache, value_center=None,
            sm_scale: Optional[float] = None, out=None, lse=None, return_lse: bool = False,
            finalize: Optional[tuple] = None):
        """``finalize=(positions, code_pages_per_request)``: also finalize the
        page that the token at ``positions`` (device int32, one per request,
        or one shared) completed, into ``codes`` and the page scales
        (``pg_decode_run_finalize``; the cache update then ran without it)."""
        if not self._state.planned:
            raise RuntimeError("plan() must be called before run()")
        k_codes, v_codes = codes
        exact_k, exact_v = exact_cache
        _check_query(q, self._batch, self._num_qo_heads)
        _check_cache(k_codes, "k_codes", torch.int8, self._num_kv_heads)
        _check_cache(v_codes, "v_codes", torch.int8, self._num_kv_heads)
        _check_scale(k_page_scale, "k_page_scale", k_codes.size(0), self._num_kv_heads)
        _check_scale(v_page_scale, "v_page_scale", v_codes.size(0), self._num_kv_heads)
        _check_cache(exact_k, "exact_k", torch.float16, self._num_kv_heads)
        _check_cache(exact_v, "exact_v", torch.float16, self._num_kv_heads)
        _check_page_ids(self._id_ranges[0], min(k_codes.size(0), v_codes.size(0)), "INT8")
        _check_page_ids(self._id_ranges[1], min(exact_k.size(0), exact_v.size(0)), "exact tail")
        center_stride = 0
        if value_center is not None:
            if (not value_center.is_cuda or value_center.dtype != torch.float16
                    or not value_center.is_contiguous()):
                raise ValueError("value_center must be contiguous CUDA float16")
            if value_center.dim() == 3 and tuple(value_center.shape) == (self._batch, self._num_kv_heads, DIM):
                center_stride = self._num_kv_heads * DIM
            elif not (value_center.dim() == 2 and self._batch == 1
                      and tuple(value_center.shape) == (self._num_kv_heads, DIM)):
                raise ValueError("value_center must be [B,Hkv,128] (or [Hkv,128] for batch one)")
        if out is None:
            out = torch.empty_like(q)
        if return_lse and lse is None:
            lse = torch.empty(q.size(0), q.size(1), device=q.device, dtype=torch.float32)
        scale = self._sm_scale if sm_scale is None else sm_scale
        args = (ctypes.byref(self._state.plan), q.data_ptr(), q.stride(0), k_codes.data_ptr(),
                v_codes.data_ptr(), k_page_scale.data_ptr(), v_page_scale.data_ptr(),
                self._old[0].data_ptr(), self._old[1].data_ptr(), exact_k.data_ptr(),
                exact_v.data_ptr(), self._tail[0].data_ptr(), self._tail[1].data_ptr(),
                _ptr(value_center), center_stride, out.data_ptr(), _ptr(lse), float(scale),
                self._state.workspace.data_ptr())
        if finalize is None:
            _capi.call("pg_decode_run", *args, _stream())
        else:
            positions, stride, code_pages = _finalize_args(finalize, self._batch, k_codes.size(0))
            _capi.call("pg_decode_run_finalize", *args, positions.data_ptr(), stride, code_pages,
                       _stream())
        return (out, lse) if return_lse else out

    def bind(self, q, codes, k_page_scale, v_page_scale, exact_cache, value_center=None,
             sm_scale: Optional[float] = None, out=None, lse=None,
             stream: Optional[int] = None) -> BoundDecode:
        """Resolve a ``run`` once (validating it); see ``BoundDecode``."""
        if out is None:
            raise ValueError("bind needs a preallocated out tensor")
        self.run(q, codes, k_page_scale, v_page_scale, exact_cache, value_center, sm_scale,
                 out=out, lse=lse)
        k_codes, v_codes = codes
        exact_k, exact_v = exact_cache
        center_stride = self._num_kv_heads * DIM if (value_center is not None and value_center.dim() == 3) else 0
        scale = self._sm_scale if sm_scale is None else sm_scale
        partial = (q.data_ptr(), q.stride(0), k_codes.data_ptr(), v_codes.data_ptr(),
                   k_page_scale.data_ptr(), v_page_scale.data_ptr(), self._old[0].data_ptr(),
                   self._old[1].data_ptr(), exact_k.data_ptr(), exact_v.data_ptr(),
                   self._tail[0].data_ptr(), self._tail[1].data_ptr(), float(scale))
        combine = (_ptr(value_center), center_stride, out.data_ptr(), _ptr(lse))
        keep = (q, k_codes, v_codes, k_page_scale, v_page_scale, exact_k, exact_v, *self._old,
                *self._tail, value_center, out, lse)
        return BoundDecode(self._state, partial, combine, _stream() if stream is None else stream,
                           keep)


def validate_heterogeneous_run_inputs(query, old_k_cache, old_v_cache, k_page_scale, v_page_scale,
                                      exact_k_cache, exact_v_cache, old_kv_len,
                                      value_center) -> None:
    """The reference's ABI checks (scripts/page_gauge_heterogeneous_fa2.py:286-333),
    same messages.  The page-alignment check reads ``old_kv_len`` on the host."""
    batch = int(query.shape[0]) if query.ndim == 3 else -1
    if tuple(query.shape) != (batch, HQ, DIM) or query.dtype != torch.float16:
        raise ValueError(f"query must have decode-only shape [B,{HQ},{DIM}] and dtype float16")
    if query.device.type != "cuda" or not query.is_contiguous():
        raise ValueError("query must be contiguous CUDA storage")
    for name, cache, dtype in (("old_k_cache", old_k_cache, torch.int8),
                               ("old_v_cache", old_v_cache, torch.int8),
                               ("exact_k_cache", exact_k_cache, torch.float16),
                               ("exact_v_cache", exact_v_cache, torch.float16)):
        if (cache.device.type != "cuda" or cache.dtype != dtype or cache.ndim != 4
                or tuple(cache.shape[1:]) != (PAGE, HKV, DIM) or not cache.is_contiguous()):
            raise ValueError(f"{name} must be contiguous CUDA [{name.split('_')[0]}_pages,16,8,128] "
                             f"{dtype}")
    if old_k_cache.shape != old_v_cache.shape or exact_k_cache.shape != exact_v_cache.shape:
        raise ValueError("K/V cache shapes must match within each representation")
    for name, scale in (("k_page_scale", k_page_scale), ("v_page_scale", v_page_scale)):
        if (scale.device.type != "cuda" or scale.dtype != torch.float16
                or tuple(scale.shape) != (old_k_cache.shape[0], HKV) or not scale.is_contiguous()):
            raise ValueError(f"{name} must be contiguous CUDA [old_pages,{HKV}] float16")
    if (old_kv_len.device.type != "cuda" or old_kv_len.dtype != torch.int32
            or tuple(old_kv_len.shape) != (batch,) or not old_kv_len.is_contiguous()):
        raise ValueError("old_kv_len must be contiguous CUDA [B] int32")
    if bool(torch.any(old_kv_len % PAGE).item()):
        raise ValueError(f"old_kv_len must be page-aligned ({PAGE} tokens)")
    if (value_center.device.type != "cuda" or value_center.dtype != torch.float16
            or tuple(value_center.shape) != (batch, HKV, DIM) or not value_center.is_contiguous()):
        raise ValueError(f"value_center must be contiguous CUDA [B,{HKV},{DIM}] float16")


class HeterogeneousDecodeWrapper:
    """One-launch decode over a unified page table (INT8 history pages then
    FP16 exact pages per request): ``make_heterogeneous_page_gauge_wrapper``
    of scripts/page_gauge_heterogeneous_fa2.py:159-205 with its ``plan`` /
    ``run`` contract (:240-283, :336-381).

    ``plan(indptr, indices, last_page_len, 32, 8, 128, 16, ...)`` cuts the
    unified table into work items without knowing the INT8/FP16 boundary;
    ``run(q, (old_k, old_v), k_page_scale, v_page_scale, exact_k, exact_v,
    old_kv_len, value_center, sm_scale, out=, lse=)`` reads ``old_kv_len``
    (page aligned, device int32 [B]) on the GPU, so a caller may move the
    boundary in place between runs.  Entries below the boundary index the
    code pool, the others the exact FP16 pages.
    """

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, **_unused) -> None:
        if kv_layout != "NHD":
            raise ValueError("only the NHD layout is supported")
        self._state = _Planned(float_workspace_buffer)
        self.use_cuda_graph = use_cuda_graph

    def plan(self, indptr, indices, last_page_len, num_qo_heads: int = HQ,
             num_kv_heads: int = HKV, head_dim: int = DIM, page_size: int = PAGE,
             pos_encoding_mode: str = "NONE", q_data_type=torch.float16,
             kv_data_type=torch.int8, o_data_type=torch.float16, sm_scale=None,
             fixed_split_size: Optional[int] = None, num_cus: Optional[int] = None,
             exact_tail_pages_hint: int = 0, **_unused) -> None:
        """``exact_tail_pages_hint`` (a builder addition): how many trailing
        pages of each request's table are expected to be FP16 exact pages at
        run time; the planner gives them their own work items, weighted as
        FP16 pages.  It only balances the work; ``old_kv_len`` still decides
        the boundary at run time."""
        if pos_encoding_mode != "NONE":
            raise ValueError("only pos_encoding_mode='NONE' is supported")
        if kv_data_type != torch.int8 or q_data_type != torch.float16 or o_data_type != torch.float16:
            raise ValueError("the heterogeneous decode takes fp16 queries/outputs over int8 history")
        _check_index(indices, "indices")
        _check_index(last_page_len, "last_page_len")
        host_indptr, host_last = _host_tables(indptr, last_page_len, indices)
        self._state.make_plan(host_indptr, host_last, _capi.PG_KV_HETEROGENEOUS,
                              None, None, num_qo_heads, num_kv_heads, head_dim, page_size,
                              fixed_split_size or 0, 0, indices.device, num_cus,
                              exact_tail_pages_hint)
        self._indices = indices
        self._last_page_len = last_page_len
        self._host_indptr = host_indptr
        self._batch = host_indptr.numel() - 1
        self._num_qo_heads = num_qo_heads
        self._num_kv_heads = num_kv_heads
        self._sm_scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(head_dim)

    @property
    def split_pages(self) -> int:
        return self._state.split_pages

    @property
    def num_work_items(self) -> int:
        return self._state.num_items

    def _check_unified_page_ids(self, old_kv_len, code_pages: int, exact_pages: int) -> None:
        """Opt-in bounds check of the unified table: entries below each
        request's boundary index the code pool, the rest the exact pages.
        Reads ``old_kv_len`` on the host (a synchronisation: debug only)."""
        if not CHECK_PAGE_IDS:
            return
        ids = self._indices.detach().to("cpu")
        boundary = old_kv_len.detach().to("cpu") // PAGE
        for b in range(self._batch):
            lo, hi = int(self._host_indptr[b]), int(self._host_indptr[b + 1])
            cut = min(hi, lo + max(int(boundary[b]), 0))
            _check_page_ids(_page_id_range(ids, torch.tensor([lo, cut])), code_pages, "INT8")
            _check_page_ids(_page_id_range(ids, torch.tensor([cut, hi])), exact_pages, "exact")

    def run(self, q, paged_kv_cache, k_page_scale, v_page_scale, exact_k_cache, exact_v_cache,
            old_kv_len, value_center, sm_scale: Optional[float] = None, out=None, lse=None,
            return_lse: bool = False, finalize: Optional[tuple] = None, **_unused):
        """``finalize=(positions, code_pages_per_request)``: also finalize the
        page that the token at ``positions`` (device int32, one per request,
        or one shared) completed (``pg_decode_run_heterogeneous_finalize``)."""
        if not self._state.planned:
            raise RuntimeError("plan() must be called before run()")
        old_k, old_v = paged_kv_cache
        _check_query(q, self._batch, self._num_qo_heads)
        _check_cache(old_k, "old_k_cache", torch.int8, self._num_kv_heads)
        _check_cache(old_v, "old_v_cache", torch.int8, self._num_kv_heads)
        _check_scale(k_page_scale, "k_page_scale", old_k.size(0), self._num_kv_heads)
        _check_scale(v_page_scale, "v_page_scale", old_v.size(0), self._num_kv_heads)
        _check_cache(exact_k_cache, "exact_k_cache", torch.float16, self._num_kv_heads)
        _check_cache(exact_v_cache, "exact_v_cache", torch.float16, self._num_kv_heads)
        _check_index(old_kv_len, "old_kv_len")
        if old_kv_len.numel() != self._batch:
            raise ValueError("old_kv_len must be contiguous CUDA [B] int32")
        self._check_unified_page_ids(old_kv_len, min(old_k.size(0), old_v.size(0)),
                                     min(exact_k_cache.size(0), exact_v_cache.size(0)))
        if (value_center.dtype != torch.float16 or not value_center.is_contiguous()
                or tuple(value_center.shape) != (self._batch, self._num_kv_heads, DIM)):
            raise ValueError("value_center must be contiguous CUDA [B,Hkv,128] float16")
        if out is None:
            out = torch.empty_like(q)
        if return_lse and lse is None:
            lse = torch.empty(q.size(0), q.size(1), device=q.device, dtype=torch.float32)
        scale = self._sm_scale if sm_scale is None else float(sm_scale)
        args = (ctypes.byref(self._state.plan), q.data_ptr(), q.stride(0), old_k.data_ptr(),
                old_v.data_ptr(), k_page_scale.data_ptr(), v_page_scale.data_ptr(),
                exact_k_cache.data_ptr(), exact_v_cache.data_ptr(), self._indices.data_ptr(),
                self._last_page_len.data_ptr(), old_kv_len.data_ptr(), value_center.data_ptr(),
                self._num_kv_heads * DIM, out.data_ptr(), _ptr(lse), scale,
                self._state.workspace.data_ptr())
        if finalize is None:
            _capi.call("pg_decode_run_heterogeneous", *args, _stream())
        else:
            positions, stride, code_pages = _finalize_args(finalize, self._batch, old_k.size(0))
            _capi.call("pg_decode_run_heterogeneous_finalize", *args, positions.data_ptr(), stride,
                       code_pages, _stream())
        return (out, lse) if return_lse else out


def make_heterogeneous_page_gauge_wrapper(flashinfer_module, workspace: torch.Tensor,
                                          **wrapper_kwargs) -> HeterogeneousDecodeWrapper:
    """scripts/page_gauge_heterogeneous_fa2.py:159-205; the first argument (the
    flashinfer module in the reference) is ignored."""
    if not workspace.is_cuda or workspace.dtype != torch.uint8:
        raise ValueError("workspace must be a CUDA uint8 tensor")
    wrapper = HeterogeneousDecodeWrapper(workspace, "NHD", **wrapper_kwargs)
    wrapper.page_gauge_module_uri = "pagegauge_amd/libpagegauge_hip.so:heterogeneous"
    return wrapper


def merge_state_in_place(v: torch.Tensor, s: torch.Tensor, v_other: torch.Tensor,
                         s_other: torch.Tensor, mask: Optional[torch.Tensor] = None) -> None:
    """flashinfer.merge_state_in_place (base-2 LSE) on the HIP stream."""
    for t, n in ((v, "v"), (v_other, "v_other")):
        if not t.is_cuda or t.dtype != torch.float16 or not t.is_contiguous() or t.dim() != 3:
            raise ValueError(f"{n} must be a contiguous CUDA float16 [seq, heads, dim] tensor")
    for t, n in ((s, "s"), (s_other, "s_other")):
        if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous CUDA float32 [seq, heads] tensor")
    if v.shape != v_other.shape or tuple(s.shape) != tuple(v.shape[:2]) or s.shape != s_other.shape:
        raise ValueError("merge_state shapes disagree")
    mask_u8 = None
    if mask is not None:
        mask_u8 = mask.to(device=v.device, dtype=torch.uint8).contiguous()
    _capi.call("pg_merge_state_in_place", v.data_ptr(), s.data_ptr(), v_other.data_ptr(),
               s_other.data_ptr(), _ptr(mask_u8), v.size(0), v.size(1), v.size(2), _stream())


def segment_page_table(pages_per_row: Sequence[int], tail_pages: int, sink_pages: int = 0,
                       device="cuda"):
    """Compact INT8-middle and exact sink+tail tables (identity storage).

    scripts/benchmark_flashinfer_page_affine_int8.py:392-420: returns
    (old_indptr, old_indices, exact_indptr, exact_indices) as int32 tensors.
    """
    old_counts = [max(count - tail_pages - sink_pages, 0) for count in pages_per_row]
    old_indices: list[int] = []
    exact_indices: list[int] = []
    start = 0
    for count, old in zip(pages_per_row, old_counts):
        middle = start + sink_pages
        old_indices.extend(range(middle, middle + old))
        exact_indices.extend(range(start, middle))
        exact_indices.extend(range(middle + old, start + count))
        start += count
    exact_counts = [count - old for count, old in zip(pages_per_row, old_counts)]

    def indptr(counts):
        total, out = 0, [0]
        for c in counts:
            total += c
            out.append(total)
        return torch.tensor(out, dtype=torch.int32, device=device)

    return (indptr(old_counts), torch.tensor(old_indices, dtype=torch.int32, device=device),
            indptr(exact_counts), torch.tensor(exact_indices, dtype=torch.int32, device=device))
