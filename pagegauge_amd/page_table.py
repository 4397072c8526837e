"""Page-table algebra of the PageGauge decoder harness.

Host-side integer logic that partitions a context into exact prefix (sink),
optional static exact suffix, INT8 "old" pages and the FP16 tail ring, and
writes the compact int32 tables the decode kernels read.  Same names,
arguments and error messages as
``scripts/benchmark_page_gauge_transformer.py:383-749``; pinned by the golden
lists of ``tests/test_page_gauge_transformer.py:100-216`` of the reference.
Tables are torch int32 tensors on any device (the writers copy in place so a
captured decode graph keeps reading the same storage).
"""

from __future__ import annotations

from typing import Any, Optional

import torch

PAGE = 16


def request_major_page_table(batch_size: int, logical_page_capacity: int,
                             physical_pages_per_request: Optional[int] = None,
                             device="cuda") -> torch.Tensor:
    """[B, P] map of logical pages to request-major physical storage (:383-405).

    With ``physical_pages_per_request`` < P the logical pages wrap (a ring).
    """
    if batch_size <= 0 or logical_page_capacity <= 0:
        raise ValueError("batch size and page capacity must be positive")
    per_request = logical_page_capacity if physical_pages_per_request is None else physical_pages_per_request
    if per_request <= 0:
        raise ValueError("physical pages per request must be positive")
    logical = torch.arange(logical_page_capacity, dtype=torch.int32, device=device)
    base = torch.arange(batch_size, dtype=torch.int32, device=device) * per_request
    return base[:, None] + (logical % per_request)[None, :]


def validate_exact_prefix_pages(exact_prefix_pages: int) -> int:
    if not isinstance(exact_prefix_pages, int) or exact_prefix_pages < 0:
        raise ValueError("exact prefix pages must be a nonnegative integer")
    return int(exact_prefix_pages)


def validate_exact_static_suffix_pages(exact_static_suffix_pages: int, *,
                                       exact_prefix_pages: int = 0,
                                       initial_context_pages: Optional[int] = None) -> int:
    if not isinstance(exact_static_suffix_pages, int) or exact_static_suffix_pages < 0:
        raise ValueError("exact static suffix pages must be a nonnegative integer")
    if exact_static_suffix_pages:
        if initial_context_pages is None or initial_context_pages <= 0:
            raise ValueError("an exact static suffix requires positive initial context pages")
        if exact_prefix_pages + exact_static_suffix_pages >= initial_context_pages:
            raise ValueError("fixed exact prefix and suffix must leave an initial old-cache page")
    return int(exact_static_suffix_pages)


def validate_exact_sink_pages(exact_sink_pages: int) -> int:
    """Legacy S0/S1 validator (sink of 0 or 1 page)."""
    if exact_sink_pages not in (0, 1):
        raise ValueError("exact sink pages must be 0 or 1")
    return int(exact_sink_pages)


def validate_exact_prefix_attention_path(exact_prefix_pages: int, tail_attention: str) -> int:
    exact_prefix_pages = validate_exact_prefix_pages(exact_prefix_pages)
    if exact_prefix_pages and tail_attention != "flashinfer_merge":
        raise ValueError("exact prefix pages require the segmented flashinfer_merge path")
    return exact_prefix_pages


def _suffix_begin(exact_static_suffix_pages: int, initial_context_pages: Optional[int]):
    if not exact_static_suffix_pages:
        return None
    return int(initial_context_pages) - exact_static_suffix_pages


def exact_physical_page_index(request: int, logical_page: int, exact_tail_pages: int,
                              exact_sink_pages: int = 0, exact_static_suffix_pages: int = 0,
                              initial_context_pages: Optional[int] = None) -> int:
    """Physical exact-ring slot of one logical page (:455-489).

    Storage per request: [prefix slots][static suffix slots][tail ring].
    """
    exact_sink_pages = validate_exact_prefix_pages(exact_sink_pages)
    exact_static_suffix_pages = validate_exact_static_suffix_pages(
        exact_static_suffix_pages, exact_prefix_pages=exact_sink_pages,
        initial_context_pages=initial_context_pages)
    if request < 0 or logical_page < 0 or exact_tail_pages <= 0:
        raise ValueError("exact page mapping inputs must be non-negative with a tail")
    fixed = exact_sink_pages + exact_static_suffix_pages
    suffix_begin = _suffix_begin(exact_static_suffix_pages, initial_context_pages)
    if logical_page < exact_sink_pages:
        local = logical_page
    elif suffix_begin is not None and suffix_begin <= logical_page < int(initial_context_pages):
        local = exact_sink_pages + logical_page - suffix_begin
    else:
        local = fixed + logical_page % exact_tail_pages
    return request * (fixed + exact_tail_pages) + local


def request_major_exact_page_table(batch_size: int, logical_page_capacity: int,
                                   exact_tail_pages: int, exact_sink_pages: int = 0,
                                   exact_static_suffix_pages: int = 0,
                                   initial_context_pages: Optional[int] = None,
                                   device="cuda") -> torch.Tensor:
    """[B, P] exact-slot table for every logical page (:492-524)."""
    exact_sink_pages = validate_exact_prefix_pages(exact_sink_pages)
    exact_static_suffix_pages = validate_exact_static_suffix_pages(
        exact_static_suffix_pages, exact_prefix_pages=exact_sink_pages,
        initial_context_pages=initial_context_pages)
    if batch_size <= 0 or logical_page_capacity <= 0 or exact_tail_pages <= 0:
        raise ValueError("batch, logical capacity, and exact tail must be positive")
    if exact_sink_pages >= logical_page_capacity:
        raise ValueError("exact prefix must be smaller than logical page capacity")
    logical = torch.arange(logical_page_capacity, dtype=torch.int32, device=device)
    fixed = exact_sink_pages + exact_static_suffix_pages
    local = fixed + logical % exact_tail_pages
    if exact_sink_pages:
        local = torch.where(logical < exact_sink_pages, logical, local)
    suffix_begin = _suffix_begin(exact_static_suffix_pages, initial_context_pages)
    if suffix_begin is not None:
        in_suffix = (logical >= suffix_begin) & (logical < int(initial_context_pages))
        local = torch.where(in_suffix, exact_sink_pages + logical - suffix_begin, local)
    base = torch.arange(batch_size, dtype=torch.int32, device=device) * (fixed + exact_tail_pages)
    return base[:, None] + local[None, :].to(torch.int32)


def page_gauge_logical_partition(total_pages: int, exact_tail_pages: int, exact_sink_pages: int,
                                 last_page_len: int, exact_static_suffix_pages: int = 0,
                                 initial_context_pages: Optional[int] = None) -> dict[str, Any]:
    """Exact-once prefix / static suffix / old / tail partition (:527-587)."""
    exact_sink_pages = validate_exact_prefix_pages(exact_sink_pages)
    exact_static_suffix_pages = validate_exact_static_suffix_pages(
        exact_static_suffix_pages, exact_prefix_pages=exact_sink_pages,
        initial_context_pages=initial_context_pages)
    if total_pages <= 0 or exact_tail_pages <= 0:
        raise ValueError("total and exact-tail page counts must be positive")
    if not 1 <= last_page_len <= PAGE:
        raise ValueError("last page length lies outside one page")
    tail_begin = total_pages - exact_tail_pages
    if tail_begin <= exact_sink_pages:
        raise ValueError("context must contain at least one quantized old page")
    prefix = tuple(range(exact_sink_pages))
    suffix_begin = _suffix_begin(exact_static_suffix_pages, initial_context_pages)
    suffix = tuple(range(suffix_begin, int(initial_context_pages))) if suffix_begin is not None else ()
    tail = tuple(range(tail_begin, total_pages))
    exact_set = set(prefix) | set(suffix) | set(tail)
    old = tuple(p for p in range(total_pages) if p not in exact_set)
    exact = tuple(p for p in range(total_pages) if p in exact_set)
    union = old + exact
    disjoint = len(set(union)) == len(union) and set(union) == set(range(total_pages))
    context_tokens = (total_pages - 1) * PAGE + last_page_len
    old_tokens = len(old) * PAGE
    exact_tokens = context_tokens - old_tokens
    if not disjoint or old_tokens + exact_tokens != context_tokens:
        raise RuntimeError("PageGauge logical partition is not exact and disjoint")
    return {
        "prefix_logical_pages": prefix,
        "sink_logical_pages": prefix,
        "static_suffix_logical_pages": suffix,
        "old_logical_pages": old,
        "tail_logical_pages": tail,
        "exact_logical_pages": exact,
        "tail_logical_begin": tail_begin,
        "old_page_count": len(old),
        "exact_page_count": len(exact),
        "old_token_count": old_tokens,
        "exact_token_count": exact_tokens,
        "context_token_count": context_tokens,
        "coverage_disjoint": disjoint,
    }


def write_exact_prefix_tail_page_table(destination: torch.Tensor,
                                       logical_to_exact_physical: torch.Tensor,
                                       tail_logical_begin: int, total_page_count: int,
                                       exact_sink_pages: int, exact_static_suffix_pages: int = 0,
                                       initial_context_pages: Optional[int] = None) -> torch.Tensor:
    """Prefix slots, static suffix, then the chronological tail (:590-647)."""
    exact_sink_pages = validate_exact_prefix_pages(exact_sink_pages)
    exact_static_suffix_pages = validate_exact_static_suffix_pages(
        exact_static_suffix_pages, exact_prefix_pages=exact_sink_pages,
        initial_context_pages=initial_context_pages)
    if destination.dtype != torch.int32 or logical_to_exact_physical.dtype != torch.int32:
        raise ValueError("exact page tables must use int32 indices")
    if destination.dim() != 2 or logical_to_exact_physical.dim() != 2:
        raise ValueError("exact page tables must have shape [B,P]")
    if destination.shape[0] != logical_to_exact_physical.shape[0]:
        raise ValueError("exact page-table batch sizes differ")
    if not exact_sink_pages <= tail_logical_begin < total_page_count:
        raise ValueError("exact prefix and tail logical ranges overlap or are empty")
    if total_page_count > logical_to_exact_physical.shape[1]:
        raise ValueError("exact logical page table exceeds allocated capacity")
    suffix_begin = _suffix_begin(exact_static_suffix_pages, initial_context_pages)
    tail_pages = [p for p in range(tail_logical_begin, total_page_count)
                  if not (suffix_begin is not None and suffix_begin <= p < int(initial_context_pages))]
    active = exact_sink_pages + exact_static_suffix_pages + len(tail_pages)
    if active > destination.shape[1]:
        raise ValueError("exact active table exceeds destination capacity")
    if exact_sink_pages:
        destination[:, :exact_sink_pages].copy_(logical_to_exact_physical[:, :exact_sink_pages])
    cursor = exact_sink_pages
    if suffix_begin is not None:
        destination[:, cursor:cursor + exact_static_suffix_pages].copy_(
            logical_to_exact_physical[:, suffix_begin:int(initial_context_pages)])
        cursor += exact_static_suffix_pages
    if tail_pages:
        idx = torch.tensor(tail_pages, dtype=torch.long, device=logical_to_exact_physical.device)
        destination[:, cursor:active].copy_(logical_to_exact_physical.index_select(1, idx))
    return destination[:, :active]


def write_page_gauge_old_page_table(destination: torch.Tensor, logical_to_physical: torch.Tensor,
                                    old_logical_pages: tuple[int, ...]) -> torch.Tensor:
    """Write an exact-once old-page set in logical order (:650-674)."""
    if destination.dtype != torch.int32 or logical_to_physical.dtype != torch.int32:
        raise ValueError("old page tables must use int32 indices")
    if destination.dim() != 2 or logical_to_physical.dim() != 2:
        raise ValueError("old page tables must have shape [B,P]")
    if destination.shape[0] != logical_to_physical.shape[0]:
        raise ValueError("old page-table batch sizes differ")
    if not old_logical_pages:
        raise ValueError("old page set cannot be empty")
    if tuple(sorted(set(old_logical_pages))) != tuple(old_logical_pages):
        raise ValueError("old logical pages must be unique and increasing")
    if old_logical_pages[-1] >= logical_to_physical.shape[1]:
        raise ValueError("old logical page exceeds allocated capacity")
    if len(old_logical_pages) > destination.shape[1]:
        raise ValueError("old page set exceeds destination capacity")
    idx = torch.tensor(old_logical_pages, dtype=torch.long, device=logical_to_physical.device)
    destination[:, :len(old_logical_pages)].copy_(logical_to_physical.index_select(1, idx))
    return destination[:, :len(old_logical_pages)]


def write_exact_sink_tail_page_table(destination: torch.Tensor,
                                     logical_to_exact_physical: torch.Tensor,
                                     tail_logical_begin: int, total_page_count: int,
                                     exact_sink_pages: int) -> torch.Tensor:
    """Legacy name of ``write_exact_prefix_tail_page_table`` (:677-692)."""
    return write_exact_prefix_tail_page_table(destination, logical_to_exact_physical,
                                              tail_logical_begin, total_page_count,
                                              exact_sink_pages)


def write_heterogeneous_page_table(destination: torch.Tensor, old_pages: torch.Tensor,
                                   exact_ring_pages: torch.Tensor, old_page_count: int,
                                   total_page_count: int) -> torch.Tensor:
    """One table over INT8 storage (< old_page_count) then the exact ring (:695-727)."""
    if destination.dtype != torch.int32:
        raise ValueError("heterogeneous page table must use int32 indices")
    if (destination.dim() != 2 or old_pages.shape != destination.shape
            or exact_ring_pages.shape != destination.shape):
        raise ValueError("heterogeneous page tables must have matching [B,P] shapes")
    if not 0 <= old_page_count <= total_page_count <= destination.shape[1]:
        raise ValueError("heterogeneous page counts lie outside table capacity")
    if old_page_count:
        destination[:, :old_page_count].copy_(old_pages[:, :old_page_count])
    if old_page_count < total_page_count:
        destination[:, old_page_count:total_page_count].copy_(
            exact_ring_pages[:, old_page_count:total_page_count])
    return destination[:, :total_page_count]


def flatten_page_table(table: torch.Tensor, pages_per_request) -> tuple[torch.Tensor, torch.Tensor]:
    """[B, P] table + per-request page counts -> (indptr [B+1], indices) int32."""
    counts = [int(c) for c in pages_per_request]
    if len(counts) != table.shape[0]:
        raise ValueError("one page count per request is required")
    if any(c < 0 or c > table.shape[1] for c in counts):
        raise ValueError("page counts lie outside the table")
    indices = torch.cat([table[r, :c] for r, c in enumerate(counts)]) if counts else table[:0, 0]
    indptr = [0]
    for c in counts:
        indptr.append(indptr[-1] + c)
    return (torch.tensor(indptr, dtype=torch.int32, device=table.device),
            indices.to(torch.int32).contiguous())
