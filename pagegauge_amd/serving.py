"""Serving metadata for PageGauge decode batches: per-request ragged
positions, a shared physical page pool and per-request exact sidecars.

Host restatement of the reference's serving prototype
(experiments/mlsys2027/serving_v1/pagegauge_vllm/): the page-aligned
prefix/suffix/tail policy (``partition.py:1-52``), request slots with leases
and generations (``request_slots.py:1-93``), decode-batch metadata
(``decode_metadata.py:1-76``) and pool accounting (``cache_layout.py:1-38``,
``sidecars.py:1-35``), with the same validation messages.  What the reference
leaves open ("GPU integration must encode evicted exact pages before
overwriting ring slots", decode_metadata.py:1-5) is here:

* ``decode_tables`` turns a prepared ``DecodeBatch`` into the device tensors
  of one step: per-row positions and the exact / code page of each row's
  token for ``rope_append_page_gauge_slots`` (K2; a page is quantised into its
  code page when its 16th token lands, so every page that later ages out of
  the tail ring already has codes), and the INT8-history and exact CSR tables
  for ``PageGaugeSegmentedDecode`` (K1);
* ``dense_pool_views`` / ``from_engine_layer`` / ``zero_physical_pages`` /
  ``allocate_sidecars`` give the pools and sidecars in the layouts the kernels
  read (cache_views.py:1-62).

The request lifecycle and scheduler transactions built on ``RequestSlots``
are in ``serving_bridge``.  CPU bookkeeping only; streams and events are the
caller's.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass
from typing import Any

PAGE = 16


@dataclass(frozen=True)
class Policy:
    """Exact prefix S, exact static suffix A (last prompt pages) and FP16
    tail ring T, in pages (partition.py:8-20)."""

    prefix_pages: int = 4
    suffix_pages: int = 128
    tail_pages: int = 48

    def __post_init__(self) -> None:
        values = (self.prefix_pages, self.suffix_pages, self.tail_pages)
        if (any(type(v) is not int for v in values) or min(self.prefix_pages, self.suffix_pages) < 0
                or self.tail_pages < 1):
            raise ValueError("Invalid page policy")

    @property
    def storage_pages(self) -> int:
        return self.prefix_pages + self.suffix_pages + self.tail_pages


def partition(prompt_tokens: int, current_tokens: int, policy: Policy = Policy()) -> dict:
    """Exact-once split of a request's pages (partition.py:23-40).  The
    partial prefill page belongs to the tail; the last (possibly partial)
    page is never history."""
    if (type(prompt_tokens) is not int or type(current_tokens) is not int
            or not 0 < prompt_tokens <= current_tokens):
        raise ValueError("Invalid prompt/current length")
    initial = prompt_tokens // PAGE
    pages = (current_tokens + PAGE - 1) // PAGE
    if (initial < policy.prefix_pages + policy.suffix_pages
            or pages - policy.tail_pages <= policy.prefix_pages):
        raise ValueError("Prompt cannot support this policy; explicit FP16 fallback required")
    prefix = range(policy.prefix_pages)
    suffix = range(initial - policy.suffix_pages, initial)
    tail = range(pages - policy.tail_pages, pages)
    exact = sorted(set(prefix) | set(suffix) | set(tail))
    exact_set = set(exact)
    history = [p for p in range(pages) if p not in exact_set]
    if not history or pages - 1 in history:
        raise ValueError("No historical page or partial last page incorrectly quantized")
    return {"prefix": tuple(prefix), "suffix": tuple(suffix), "tail": tuple(tail),
            "exact": tuple(exact), "history": tuple(history),
            "history_tokens": PAGE * len(history),
            "exact_tokens": current_tokens - PAGE * len(history),
            "tail_tokens": (policy.tail_pages - 1) * PAGE + (current_tokens - 1) % PAGE + 1}


def exact_slot(logical_page: int, prompt_tokens: int, lease_slot: int,
               policy: Policy = Policy()) -> int:
    """Exact page of a logical page in the sidecar of ``lease_slot``:
    [prefix slots][suffix slots][tail ring] (partition.py:43-52)."""
    initial = prompt_tokens // PAGE
    if min(logical_page, lease_slot) < 0:
        raise ValueError("Negative page/lease slot")
    if logical_page < policy.prefix_pages:
        local = logical_page
    elif initial - policy.suffix_pages <= logical_page < initial:
        local = policy.prefix_pages + logical_page - (initial - policy.suffix_pages)
    else:
        local = policy.prefix_pages + policy.suffix_pages + logical_page % policy.tail_pages
    return lease_slot * policy.storage_pages + local


@dataclass(frozen=True)
class Lease:
    request_id: str
    slot: int
    generation: int


@dataclass(frozen=True)
class State:
    lease: Lease
    prompt_tokens: int
    current_tokens: int
    physical_pages: tuple


class RequestSlots:
    """Admission capacity, leases (slot + generation) and page ownership;
    removing a row from a batch never frees request state
    (request_slots.py:24-93)."""

    def __init__(self, maximum_requests: int, policy: Policy = Policy()) -> None:
        if type(maximum_requests) is not int or maximum_requests < 1:
            raise ValueError("Positive fixed admission capacity required")
        self.policy = policy
        self.free = list(range(maximum_requests))
        self.generations = [0] * maximum_requests
        self.states: dict[str, State] = {}
        self.page_owner: dict[int, Lease] = {}

    def clone(self) -> "RequestSlots":
        """Independent copy of the bookkeeping (leases and states are immutable,
        so the containers are all that is copied)."""
        other = RequestSlots.__new__(RequestSlots)
        other.policy = self.policy
        other.free = list(self.free)
        other.generations = list(self.generations)
        other.states = dict(self.states)
        other.page_owner = dict(self.page_owner)
        return other

    def _pages(self, physical_pages, count: int) -> tuple:
        pages = tuple(physical_pages)
        if (len(pages) != count or len(set(pages)) != count
                or any(type(p) is not int or p < 0 for p in pages)):
            raise ValueError("Wrong/duplicate physical block table")
        return pages

    def admit(self, request_id: str, prompt_tokens: int, physical_pages) -> Lease:
        if not isinstance(request_id, str) or not request_id or request_id in self.states:
            raise ValueError("Invalid or duplicate live request ID")
        partition(prompt_tokens, prompt_tokens, self.policy)
        pages = self._pages(physical_pages, (prompt_tokens + PAGE - 1) // PAGE)
        if any(p in self.page_owner for p in pages):
            raise ValueError("Cross-request page sharing is disabled")
        if not self.free:
            raise MemoryError("Declared exact-sidecar admission capacity reached")
        slot = heapq.heappop(self.free)
        self.generations[slot] += 1
        lease = Lease(request_id, slot, self.generations[slot])
        self.states[request_id] = State(lease, prompt_tokens, prompt_tokens, pages)
        self.page_owner.update((p, lease) for p in pages)
        return lease

    def state(self, lease: Lease) -> State:
        state = self.states.get(lease.request_id)
        if state is None or state.lease != lease:
            raise ValueError("Stale request lease/center generation")
        return state

    def batch(self, request_ids) -> tuple:
        ids = tuple(request_ids)
        if len(set(ids)) != len(ids):
            raise ValueError("Duplicate batch row")
        try:
            return tuple(self.states[name].lease for name in ids)
        except KeyError as error:
            raise ValueError("Unknown scheduled request") from error

    def append(self, lease: Lease, position: int, physical_pages) -> dict:
        state = self.state(lease)
        if position != state.current_tokens:
            raise ValueError("Skipped/replayed token or wrong per-request position")
        length = position + 1
        pages = self._pages(physical_pages, (length + PAGE - 1) // PAGE)
        if pages[:len(state.physical_pages)] != state.physical_pages:
            raise ValueError("Preemption/remapping is not supported in phase one")
        extra = pages[len(state.physical_pages):]
        if any(p in self.page_owner for p in extra):
            raise ValueError("New physical page belongs to a live request")
        before = partition(state.prompt_tokens, state.current_tokens, self.policy)
        after = partition(state.prompt_tokens, length, self.policy)
        aged = sorted(set(after["history"]) - set(before["history"]))
        if any(p >= length // PAGE for p in aged):
            raise ValueError("Attempt to consume an unfinished INT8 page")
        self.page_owner.update((p, lease) for p in extra)
        self.states[lease.request_id] = State(lease, state.prompt_tokens, length, pages)
        return {"lease": lease, "position": position,
                "closed_page": position // PAGE if length % PAGE == 0 else None,
                "new_history_pages": tuple(aged), "partition": after}

    def release(self, lease: Lease) -> None:
        state = self.state(lease)
        for page in state.physical_pages:
            if self.page_owner.get(page) != lease:
                raise ValueError("Page ownership corrupted")
        for page in state.physical_pages:
            del self.page_owner[page]
        del self.states[lease.request_id]
        heapq.heappush(self.free, lease.slot)


@dataclass(frozen=True)
class DecodeRow:
    lease: Lease
    expected_state: State
    position: int
    physical_pages: tuple
    physical_token_slot: int
    exact_token_slot: int
    new_history_logical_pages: tuple
    new_history_physical_pages: tuple
    new_history_exact_slots: tuple


@dataclass(frozen=True)
class DecodeBatch:
    rows: tuple

    def columns(self) -> dict:
        """Integer columns of the batch, ordered by scheduled row (decode_metadata.py:29-36)."""
        return {"request_slots": tuple(r.lease.slot for r in self.rows),
                "generations": tuple(r.lease.generation for r in self.rows),
                "positions": tuple(r.position for r in self.rows),
                "physical_token_slots": tuple(r.physical_token_slot for r in self.rows),
                "exact_token_slots": tuple(r.exact_token_slot for r in self.rows)}


def prepare_decode(manager: RequestSlots, scheduled) -> DecodeBatch:
    """Validate one decode step without mutating the manager; ``scheduled``
    holds (lease, next position, full physical block table)
    (decode_metadata.py:39-62)."""
    rows, ids, allocated = [], set(), set(manager.page_owner)
    policy = manager.policy
    for lease, position, physical_pages in scheduled:
        state = manager.state(lease)
        if lease.request_id in ids:
            raise ValueError("Duplicate scheduled request")
        ids.add(lease.request_id)
        if type(position) is not int or position != state.current_tokens:
            raise ValueError("Wrong next token position")
        pages = manager._pages(physical_pages, (position + PAGE) // PAGE)
        if pages[:len(state.physical_pages)] != state.physical_pages:
            raise ValueError("Physical remapping is unsupported")
        extra = pages[len(state.physical_pages):]
        if any(p in allocated for p in extra):
            raise ValueError("Physical page alias across batch")
        allocated.update(extra)
        before = partition(state.prompt_tokens, position, policy)
        after = partition(state.prompt_tokens, position + 1, policy)
        aged = tuple(sorted(set(after["history"]) - set(before["history"])))
        if any(p >= (position + 1) // PAGE for p in aged):
            raise ValueError("Cannot quantize incomplete page")
        page = position // PAGE
        rows.append(DecodeRow(
            lease, state, position, pages, pages[page] * PAGE + position % PAGE,
            exact_slot(page, state.prompt_tokens, lease.slot, policy) * PAGE + position % PAGE,
            aged, tuple(pages[p] for p in aged),
            tuple(exact_slot(p, state.prompt_tokens, lease.slot, policy) for p in aged)))
    return DecodeBatch(tuple(rows))


def commit_decode(manager: RequestSlots, batch: DecodeBatch) -> tuple:
    """Advance the manager after the caller has fenced the batch's GPU work;
    the whole batch is re-validated first (decode_metadata.py:65-76)."""
    for row in batch.rows:
        if manager.state(row.lease) != row.expected_state:
            raise ValueError("Decode batch is stale")
    fresh = prepare_decode(manager, [(r.lease, r.position, r.physical_pages) for r in batch.rows])
    if fresh != batch:
        raise ValueError("Decode metadata was altered")
    return tuple(manager.append(r.lease, r.position, r.physical_pages) for r in batch.rows)


@dataclass
class DecodeTables:
    """Device tensors of one decode step (int32; CSR tables per segment)."""

    positions: Any             # [B]     token position of each row
    exact_page_ids: Any        # [B]     exact page of the row's token (K2)
    code_page_ids: Any         # [B]     physical page of the row's token (K2 finalize)
    request_slots: Any         # [B]     sidecar slot of each row (centers)
    old_indptr: Any            # [B+1]   INT8 history pages (physical ids, logical order)
    old_indices: Any
    old_last_page_len: Any     # [B]     16 (history pages are whole)
    exact_indptr: Any          # [B+1]   exact pages (sidecar slots, logical order)
    exact_indices: Any
    exact_last_page_len: Any   # [B]     tokens of the row's current page after the append


def decode_tables(batch: DecodeBatch, policy: Policy, device="cuda") -> DecodeTables:
    """The K2 ids and K1 tables of a prepared batch, for the context after
    each row's token is appended (position + 1 tokens)."""
    import torch

    positions, exact_ids, code_ids, slots = [], [], [], []
    old_ptr, old_idx, exact_ptr, exact_idx, exact_last = [0], [], [0], [], []
    for row in batch.rows:
        prompt = row.expected_state.prompt_tokens
        page = row.position // PAGE
        positions.append(row.position)
        exact_ids.append(row.exact_token_slot // PAGE)
        code_ids.append(row.physical_token_slot // PAGE)
        slots.append(row.lease.slot)
        part = partition(prompt, row.position + 1, policy)
        if part["exact"][-1] != page:
            raise RuntimeError("the row's current page must be the last exact page")
        old_idx.extend(row.physical_pages[p] for p in part["history"])
        exact_idx.extend(exact_slot(p, prompt, row.lease.slot, policy) for p in part["exact"])
        old_ptr.append(len(old_idx))
        exact_ptr.append(len(exact_idx))
        exact_last.append(row.position % PAGE + 1)
    t = lambda values: torch.tensor(values, dtype=torch.int32, device=device)  # noqa: E731
    batch_size = len(batch.rows)
    return DecodeTables(t(positions), t(exact_ids), t(code_ids), t(slots), t(old_ptr), t(old_idx),
                        t([PAGE] * batch_size), t(exact_ptr), t(exact_idx), t(exact_last))


@dataclass(frozen=True)
class Layout:
    """Pool geometry and byte accounting of one served cache (cache_layout.py:7-38)."""

    layers: int
    physical_pages: int
    maximum_requests: int
    kv_heads: int = 8
    query_heads: int = 32
    head_dim: int = 128
    policy: Policy = Policy()

    def __post_init__(self) -> None:
        values = (self.layers, self.physical_pages, self.maximum_requests, self.kv_heads,
                  self.query_heads, self.head_dim)
        if any(type(v) is not int or v < 1 for v in values) or self.query_heads % self.kv_heads:
            raise ValueError("Invalid cache geometry")

    def accounting(self) -> dict:
        layers, pages, requests = self.layers, self.physical_pages, self.maximum_requests
        h, q, d = self.kv_heads, self.query_heads, self.head_dim
        storage = self.policy.storage_pages
        tensors = {"key_codes": layers * pages * PAGE * h * d,
                   "value_codes": layers * pages * PAGE * h * d,
                   "key_scales": 2 * layers * pages * h, "value_scales": 2 * layers * pages * h,
                   "exact_key": 2 * layers * requests * storage * PAGE * h * d,
                   "exact_value": 2 * layers * requests * storage * PAGE * h * d,
                   "key_center": 2 * layers * requests * h * d,
                   "value_center": 2 * layers * requests * h * d,
                   "output_center": 2 * layers * requests * q * d}
        page_pool = sum(tensors[k] for k in ("key_codes", "value_codes", "key_scales",
                                             "value_scales"))
        sidecar = sum(tensors.values()) - page_pool
        return {"tensors": tensors, "page_pool_bytes": page_pool,
                "reserved_sidecar_bytes": sidecar,
                "total_served_capacity_bytes": sum(tensors.values()),
                "per_layer_page_bytes": 2 * PAGE * h * d + 4 * h,
                "scope": "Declared persistent code/metadata pool and all admitted-request sidecar "
                         "slots, including empty reserved slots. Excludes weights, workspace, "
                         "graph pools, input/output buffers and allocator padding."}

    def admissible_pages(self, cache_budget_bytes: int) -> int:
        accounting = self.accounting()
        remaining = cache_budget_bytes - accounting["reserved_sidecar_bytes"]
        if remaining < 0:
            raise MemoryError("Budget cannot hold reserved exact/center sidecars")
        return remaining // (self.layers * accounting["per_layer_page_bytes"])


def dense_pool_views(raw, physical_pages: int, kv_heads: int, head_dim: int = 128) -> dict:
    """K/V code planes and K/V scale planes of one layer's raw uint8 pool, no
    copy (cache_views.py:9-27): the [pages,16,Hkv,128] int8 and [pages,Hkv]
    fp16 layouts K1 and K2 read."""
    import torch

    if any(type(x) is not int or x < 1 for x in (physical_pages, kv_heads, head_dim)):
        raise ValueError("Positive integer pool geometry required")
    codes = physical_pages * PAGE * kv_heads * head_dim
    scales = physical_pages * kv_heads * 2
    if (raw.dtype != torch.uint8 or raw.ndim != 1 or not raw.is_contiguous()
            or raw.numel() != 2 * codes + 2 * scales or raw.data_ptr() % 16):
        raise ValueError("Aligned contiguous uint8 layer allocation of exact size required")
    return {
        "key_codes": raw[:codes].view(torch.int8).view(physical_pages, PAGE, kv_heads, head_dim),
        "value_codes": raw[codes:2 * codes].view(torch.int8).view(physical_pages, PAGE, kv_heads,
                                                                   head_dim),
        "key_scales": raw[2 * codes:2 * codes + scales].view(torch.float16).view(physical_pages,
                                                                                 kv_heads),
        "value_scales": raw[2 * codes + scales:].view(torch.float16).view(physical_pages, kv_heads),
    }


def from_engine_layer(layer, physical_pages: int, kv_heads: int) -> dict:
    """The planes of a compact packed engine layer [pages, Hkv, 1, 2*16*128+4]
    uint8, reinterpreted in place (cache_views.py:30-41)."""
    import torch

    expected = (physical_pages, kv_heads, 1, 2 * PAGE * 128 + 4)
    if layer.dtype != torch.uint8 or tuple(layer.shape) != expected or not layer.is_contiguous():
        raise ValueError("Compact packed engine layer required; copying is forbidden")
    return dense_pool_views(layer.view(-1), physical_pages, kv_heads)


def zero_physical_pages(views: dict, page_ids) -> None:
    """Clear fresh pages in all four planes on the current stream (an index
    fill kernel per plane) before they are used (cache_views.py:44-62)."""
    import torch

    planes = tuple(views[name] for name in ("key_codes", "value_codes", "key_scales",
                                            "value_scales"))
    first = planes[0]
    pages = tuple(page_ids)
    if (any(t.device != first.device or t.shape[0] != first.shape[0] for t in planes)
            or any(type(p) is not int or not 0 <= p < first.shape[0] for p in pages)
            or len(set(pages)) != len(pages)):
        raise ValueError("Invalid physical pages or inconsistent pool views")
    if not pages:
        return
    index = torch.tensor(pages, dtype=torch.int64, device=first.device)
    for plane in planes:
        plane.index_fill_(0, index, 0)


def allocate_sidecars(layout: Layout, *, device, cache_budget_bytes: int) -> dict:
    """Exact pages and centers reserved for every admission slot
    (sidecars.py:10-35), zero-initialised."""
    import torch

    if type(cache_budget_bytes) is not int or cache_budget_bytes < 0:
        raise ValueError("Nonnegative integer cache-only byte budget required")
    accounting = layout.accounting()
    if accounting["total_served_capacity_bytes"] > cache_budget_bytes:
        raise MemoryError("Code pool plus all reserved sidecars exceed cache budget")
    exact_shape = (layout.layers, layout.maximum_requests * layout.policy.storage_pages, PAGE,
                   layout.kv_heads, layout.head_dim)
    center_shape = (layout.layers, layout.maximum_requests, layout.kv_heads, layout.head_dim)
    shapes = {"exact_key": exact_shape, "exact_value": exact_shape, "key_center": center_shape,
              "value_center": center_shape,
              "output_center": (layout.layers, layout.maximum_requests, layout.query_heads,
                                layout.head_dim)}
    result = {name: torch.zeros(shape, dtype=torch.float16, device=device)
              for name, shape in shapes.items()}
    for name, tensor in result.items():
        if tensor.numel() * tensor.element_size() != accounting["tensors"][name]:
            raise RuntimeError("Sidecar allocation differs from declared accounting")
    return result
