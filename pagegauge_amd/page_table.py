"""Page tables of the PageGauge decoder harness.

A request's context is a run of 16-token logical pages.  Each page is served
either from the INT8 code pool ("old" pages) or from the request's exact FP16
storage.  The exact storage of one request is a fixed block of slots:

    [ prefix (sink) slots | static-suffix slots | tail ring slots ]
      S pages               A pages               E pages

* the first S logical pages (the attention sink) keep slots 0..S-1;
* the A pages just before ``initial_context_pages`` (the static suffix of
  the prefill) keep slots S..S+A-1;
* every other page that is exact at some point is one of the newest E pages
  of the context and lives in ring slot ``S + A + page % E``.

``ExactPageLayout`` holds (S, A, I, E) and answers every question the
decoder asks: the slot of a page, the slot table of a whole capacity, the
partition of a context of T pages into old and exact pages, and the order in
which the exact pages are listed for the exact decode segment.  The public
functions keep the names, arguments, messages and return keys of the
reference harness's page-table helpers
(``scripts/benchmark_page_gauge_transformer.py:383-749``), whose behaviour
the golden lists of its tests pin (``tests/test_page_gauge_transformer.py:
100-216, 785-870``).  Tables are torch int32 tensors on any device; the
writers fill a caller-owned destination in place, so a captured decode graph
keeps reading the same storage.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional, Sequence

import torch

PAGE = 16


# ---------------------------------------------------------------------------
# Argument checks (the reference's conditions and messages)
# ---------------------------------------------------------------------------
def validate_exact_prefix_pages(exact_prefix_pages: int) -> int:
    """Exact prefix (attention sink) page count: a nonnegative int."""
    if isinstance(exact_prefix_pages, int) and exact_prefix_pages >= 0:
        return int(exact_prefix_pages)
    raise ValueError("exact prefix pages must be a nonnegative integer")


def validate_exact_static_suffix_pages(exact_static_suffix_pages: int, *,
                                       exact_prefix_pages: int = 0,
                                       initial_context_pages: Optional[int] = None) -> int:
    """Static-suffix page count.  A nonzero suffix needs a positive initial
    context that keeps at least one INT8 page between prefix and suffix."""
    if not isinstance(exact_static_suffix_pages, int) or exact_static_suffix_pages < 0:
        raise ValueError("exact static suffix pages must be a nonnegative integer")
    if exact_static_suffix_pages == 0:
        return 0
    if initial_context_pages is None or initial_context_pages <= 0:
        raise ValueError("an exact static suffix requires positive initial context pages")
    if initial_context_pages <= exact_prefix_pages + exact_static_suffix_pages:
        raise ValueError("fixed exact prefix and suffix must leave an initial old-cache page")
    return int(exact_static_suffix_pages)


def validate_exact_sink_pages(exact_sink_pages: int) -> int:
    """Sink of 0 or 1 page (the reference's older S0/S1 protocol)."""
    if exact_sink_pages in (0, 1):
        return int(exact_sink_pages)
    raise ValueError("exact sink pages must be 0 or 1")


def validate_exact_prefix_attention_path(exact_prefix_pages: int, tail_attention: str) -> int:
    """An exact prefix is served by the segmented path only (the fused tail
    kernel and the one-table heterogeneous decode assume a lone tail)."""
    pages = validate_exact_prefix_pages(exact_prefix_pages)
    if pages and tail_attention != "flashinfer_merge":
        raise ValueError("exact prefix pages require the segmented flashinfer_merge path")
    return pages


# ---------------------------------------------------------------------------
# The layout of one request's exact storage
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class ExactPageLayout:
    prefix: int                 # S: sink pages, slots [0, S)
    suffix: int                 # A: static-suffix pages, slots [S, S + A)
    initial: Optional[int]      # I: initial context pages (the suffix ends there)
    tail: int                   # E: ring pages, slots [S + A, S + A + E)

    @classmethod
    def checked(cls, prefix: int, suffix: int, initial: Optional[int],
                tail: int) -> "ExactPageLayout":
        """Layout after the prefix and suffix checks; callers check ``tail``
        with their own message."""
        prefix = validate_exact_prefix_pages(prefix)
        suffix = validate_exact_static_suffix_pages(suffix, exact_prefix_pages=prefix,
                                                    initial_context_pages=initial)
        return cls(prefix, suffix, None if initial is None else int(initial), tail)

    @property
    def fixed(self) -> int:
        """Slots that never move: prefix + static suffix."""
        return self.prefix + self.suffix

    @property
    def storage(self) -> int:
        """Exact slots per request."""
        return self.fixed + self.tail

    @property
    def suffix_pages(self) -> range:
        """Logical pages of the static suffix, [I - A, I)."""
        if not self.suffix:
            return range(0)
        return range(self.initial - self.suffix, self.initial)

    def slot(self, page: int) -> int:
        """Exact slot of logical page ``page`` within its request."""
        if page < self.prefix:
            return page
        span = self.suffix_pages
        if page in span:
            return self.prefix + (page - span.start)
        return self.fixed + page % self.tail

    def slots(self, capacity: int, device) -> torch.Tensor:
        """``slot`` of logical pages 0..capacity-1 as int32 [capacity]: the ring
        formula everywhere, then the prefix and suffix spans overwritten."""
        pages = torch.arange(capacity, dtype=torch.int32, device=device)
        local = pages.remainder(self.tail) + self.fixed
        head = min(self.prefix, capacity)
        local[:head] = pages[:head]
        span = self.suffix_pages
        lo, hi = span.start, min(span.stop, capacity)
        if lo < hi:
            local[lo:hi] = pages[lo:hi] - span.start + self.prefix
        return local

    def old_pages(self, total: int) -> list[int]:
        """INT8 pages of a context of ``total`` pages, increasing: the pages
        between the prefix and the tail ring, less the static suffix."""
        tail_begin = total - self.tail
        span = self.suffix_pages
        if not span:
            return list(range(self.prefix, tail_begin))
        return (list(range(self.prefix, min(span.start, tail_begin))) +
                list(range(max(span.stop, self.prefix), tail_begin)))

    def exact_order(self, tail_begin: int, total: int) -> list[int]:
        """Logical pages of the exact segment in table order: prefix, static
        suffix, then the tail pages [tail_begin, total) in time order (tail
        pages still inside the suffix are listed once, with the suffix)."""
        span = self.suffix_pages
        return (list(range(self.prefix)) + list(span) +
                [p for p in range(tail_begin, total) if p not in span])


def _request_major(batch_size: int, stride: int, local: torch.Tensor) -> torch.Tensor:
    """[B, P] table: request r's block starts at r * stride."""
    base = torch.arange(batch_size, dtype=torch.int32, device=local.device) * stride
    return base[:, None] + local[None, :]


# ---------------------------------------------------------------------------
# Logical -> physical maps
# ---------------------------------------------------------------------------
def request_major_page_table(batch_size: int, logical_page_capacity: int,
                             physical_pages_per_request: Optional[int] = None,
                             device="cuda") -> torch.Tensor:
    """[B, P] map of logical pages to request-major physical pages
    (``:383-405``).  With fewer physical pages than P the logical pages wrap
    around the request's block (a ring)."""
    if batch_size <= 0 or logical_page_capacity <= 0:
        raise ValueError("batch size and page capacity must be positive")
    block = logical_page_capacity if physical_pages_per_request is None else physical_pages_per_request
    if block <= 0:
        raise ValueError("physical pages per request must be positive")
    local = torch.arange(logical_page_capacity, dtype=torch.int32, device=device).remainder(block)
    return _request_major(batch_size, block, local)


def exact_physical_page_index(request: int, logical_page: int, exact_tail_pages: int,
                              exact_sink_pages: int = 0, exact_static_suffix_pages: int = 0,
                              initial_context_pages: Optional[int] = None) -> int:
    """Physical exact slot of one logical page (``:455-489``)."""
    layout = ExactPageLayout.checked(exact_sink_pages, exact_static_suffix_pages,
                                     initial_context_pages, exact_tail_pages)
    if min(request, logical_page) < 0 or exact_tail_pages <= 0:
        raise ValueError("exact page mapping inputs must be non-negative with a tail")
    return request * layout.storage + layout.slot(logical_page)


def request_major_exact_page_table(batch_size: int, logical_page_capacity: int,
                                   exact_tail_pages: int, exact_sink_pages: int = 0,
                                   exact_static_suffix_pages: int = 0,
                                   initial_context_pages: Optional[int] = None,
                                   device="cuda") -> torch.Tensor:
    """[B, P] exact slot of every logical page (``:492-524``)."""
    layout = ExactPageLayout.checked(exact_sink_pages, exact_static_suffix_pages,
                                     initial_context_pages, exact_tail_pages)
    if min(batch_size, logical_page_capacity, exact_tail_pages) <= 0:
        raise ValueError("batch, logical capacity, and exact tail must be positive")
    if layout.prefix >= logical_page_capacity:
        raise ValueError("exact prefix must be smaller than logical page capacity")
    return _request_major(batch_size, layout.storage, layout.slots(logical_page_capacity, device))


# ---------------------------------------------------------------------------
# Partition of a context
# ---------------------------------------------------------------------------
def page_gauge_logical_partition(total_pages: int, exact_tail_pages: int, exact_sink_pages: int,
                                 last_page_len: int, exact_static_suffix_pages: int = 0,
                                 initial_context_pages: Optional[int] = None) -> dict[str, Any]:
    """Old / exact split of a context of ``total_pages`` pages whose last page
    holds ``last_page_len`` tokens (``:527-587``).  Every page gets one class,
    so the old and exact lists cover the context exactly once."""
    layout = ExactPageLayout.checked(exact_sink_pages, exact_static_suffix_pages,
                                     initial_context_pages, exact_tail_pages)
    if total_pages <= 0 or exact_tail_pages <= 0:
        raise ValueError("total and exact-tail page counts must be positive")
    if not 1 <= last_page_len <= PAGE:
        raise ValueError("last page length lies outside one page")
    tail_begin = total_pages - exact_tail_pages
    if tail_begin <= layout.prefix:
        raise ValueError("context must contain at least one quantized old page")

    is_old = bytearray(total_pages)
    for page in layout.old_pages(total_pages):
        is_old[page] = 1
    old = tuple(p for p in range(total_pages) if is_old[p])
    exact = tuple(p for p in range(total_pages) if not is_old[p])
    tokens = (total_pages - 1) * PAGE + last_page_len
    old_tokens = PAGE * len(old)
    prefix = tuple(range(layout.prefix))
    return {
        "prefix_logical_pages": prefix,
        "sink_logical_pages": prefix,
        "static_suffix_logical_pages": tuple(layout.suffix_pages),
        "old_logical_pages": old,
        "tail_logical_pages": tuple(range(tail_begin, total_pages)),
        "exact_logical_pages": exact,
        "tail_logical_begin": tail_begin,
        "old_page_count": len(old),
        "exact_page_count": len(exact),
        "old_token_count": old_tokens,
        "exact_token_count": tokens - old_tokens,
        "context_token_count": tokens,
        "coverage_disjoint": len(old) + len(exact) == total_pages,
    }


# ---------------------------------------------------------------------------
# Active tables (written in place)
# ---------------------------------------------------------------------------
def _check_table_pair(what: str, destination: torch.Tensor, source: torch.Tensor) -> None:
    """dtype, rank and batch checks shared by the old and exact writers."""
    if destination.dtype != torch.int32 or source.dtype != torch.int32:
        raise ValueError(f"{what} page tables must use int32 indices")
    if destination.dim() != 2 or source.dim() != 2:
        raise ValueError(f"{what} page tables must have shape [B,P]")
    if destination.shape[0] != source.shape[0]:
        raise ValueError(f"{what} page-table batch sizes differ")


def _gather_columns(destination: torch.Tensor, source: torch.Tensor,
                    columns: Sequence[int]) -> torch.Tensor:
    """destination[:, j] = source[:, columns[j]]; returns the filled view."""
    index = torch.tensor(list(columns), dtype=torch.long, device=source.device)
    view = destination[:, :len(columns)]
    view.copy_(source.index_select(1, index))
    return view


def write_exact_prefix_tail_page_table(destination: torch.Tensor,
                                       logical_to_exact_physical: torch.Tensor,
                                       tail_logical_begin: int, total_page_count: int,
                                       exact_sink_pages: int, exact_static_suffix_pages: int = 0,
                                       initial_context_pages: Optional[int] = None) -> torch.Tensor:
    """Exact-segment table: prefix slots, static suffix, then the tail in time
    order (``:590-647``)."""
    layout = ExactPageLayout.checked(exact_sink_pages, exact_static_suffix_pages,
                                     initial_context_pages, 0)
    _check_table_pair("exact", destination, logical_to_exact_physical)
    if not layout.prefix <= tail_logical_begin < total_page_count:
        raise ValueError("exact prefix and tail logical ranges overlap or are empty")
    if total_page_count > logical_to_exact_physical.shape[1]:
        raise ValueError("exact logical page table exceeds allocated capacity")
    order = layout.exact_order(tail_logical_begin, total_page_count)
    if len(order) > destination.shape[1]:
        raise ValueError("exact active table exceeds destination capacity")
    return _gather_columns(destination, logical_to_exact_physical, order)


def write_page_gauge_old_page_table(destination: torch.Tensor, logical_to_physical: torch.Tensor,
                                    old_logical_pages: Sequence[int]) -> torch.Tensor:
    """INT8-segment table for a set of old pages, in logical order (``:650-674``)."""
    _check_table_pair("old", destination, logical_to_physical)
    pages = tuple(old_logical_pages)
    if not pages:
        raise ValueError("old page set cannot be empty")
    if any(b <= a for a, b in zip(pages, pages[1:])):
        raise ValueError("old logical pages must be unique and increasing")
    if pages[-1] >= logical_to_physical.shape[1]:
        raise ValueError("old logical page exceeds allocated capacity")
    if len(pages) > destination.shape[1]:
        raise ValueError("old page set exceeds destination capacity")
    return _gather_columns(destination, logical_to_physical, pages)


def write_exact_sink_tail_page_table(destination: torch.Tensor,
                                     logical_to_exact_physical: torch.Tensor,
                                     tail_logical_begin: int, total_page_count: int,
                                     exact_sink_pages: int) -> torch.Tensor:
    """Older name of ``write_exact_prefix_tail_page_table`` without a suffix
    (``:677-692``)."""
    return write_exact_prefix_tail_page_table(destination, logical_to_exact_physical,
                                              tail_logical_begin, total_page_count,
                                              exact_sink_pages)


def write_heterogeneous_page_table(destination: torch.Tensor, old_pages: torch.Tensor,
                                   exact_ring_pages: torch.Tensor, old_page_count: int,
                                   total_page_count: int) -> torch.Tensor:
    """One table per request for the heterogeneous decode (``:695-727``):
    columns below ``old_page_count`` come from the INT8 map, the rest up to
    ``total_page_count`` from the exact-ring map."""
    if destination.dtype != torch.int32:
        raise ValueError("heterogeneous page table must use int32 indices")
    if destination.dim() != 2 or not (old_pages.shape == exact_ring_pages.shape == destination.shape):
        raise ValueError("heterogeneous page tables must have matching [B,P] shapes")
    if not 0 <= old_page_count <= total_page_count <= destination.shape[1]:
        raise ValueError("heterogeneous page counts lie outside table capacity")
    for source, lo, hi in ((old_pages, 0, old_page_count),
                           (exact_ring_pages, old_page_count, total_page_count)):
        if lo < hi:
            destination[:, lo:hi].copy_(source[:, lo:hi])
    return destination[:, :total_page_count]


def flatten_page_table(table: torch.Tensor, pages_per_request) -> tuple[torch.Tensor, torch.Tensor]:
    """[B, P] table + per-request page counts -> CSR (indptr [B+1], indices) int32."""
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
