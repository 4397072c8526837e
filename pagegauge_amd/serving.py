"""Serving metadata for PageGauge decode batches: ragged per-request
positions over a shared physical page pool, with per-request exact sidecars.

The drop-in surface is the one the reference's serving prototype exposes to
its engine and pins in its tests
(experiments/mlsys2027/serving_v1/test_pinned_cache_spec.py,
test_pinned_scheduler_bridge.py): the page policy ``Policy`` with its exact
prefix S, static suffix A and FP16 tail ring T; the pool geometry ``Layout``
with its byte accounting; ``allocate_sidecars``; and the zero-copy pool views
``dense_pool_views``, ``from_engine_layer``, ``zero_physical_pages``.  The
scheduler bridge is in ``serving_bridge``.

The bookkeeping is this module's own design: one ``Ledger`` holds every
admission slot as a small state machine

    free -> prefill -> packing -> ready -> retiring -> free

together with the page-ownership table of the pool (physical page -> slot),
so admission, per-token growth, page ownership and retirement are checked in
one place.  A decode step is *staged* against the ledger without changing it
(``stage_decode``) and *committed* after the caller has fenced its GPU work
(``commit_decode``).  Every change of a slot bumps that slot's stamp and each
staged row remembers the stamp it was staged at, so a row whose request has
changed since (a committed step, a retirement, a new occupant) can never be
committed late; the pages a step adds are checked again for ownership.

What the reference leaves to "GPU integration"
(experiments/mlsys2027/serving_v1/pagegauge_vllm/decode_metadata.py:1-5) is
``decode_tables``: the device tensors of one step, i.e. per-row positions and
the exact / code page of each row's token for ``rope_append_page_gauge_slots``
(K2: a page is quantised into its physical code page when its 16th token
lands, so a page that later ages out of the tail ring already has codes) and
the INT8-history and exact CSR tables for ``PageGaugeSegmentedDecode`` (K1).

CPU bookkeeping only; streams and events are the caller's (any object with
``query()``, such as ``torch.cuda.Event``).
"""

from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Any, NamedTuple, Optional

PAGE = 16


# ---------------------------------------------------------------------------
# Page policy
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class Policy:
    """Exact pages kept per request: the first ``prefix_pages`` (S), the last
    ``suffix_pages`` whole prompt pages (A, exact for the request's life) and
    a ring of the newest ``tail_pages`` pages (T); every other page is INT8
    history (the reference's S4 / A128 / T48 default)."""

    prefix_pages: int = 4
    suffix_pages: int = 128
    tail_pages: int = 48

    def __post_init__(self) -> None:
        counts = (self.prefix_pages, self.suffix_pages, self.tail_pages)
        if not all(type(c) is int for c in counts) or min(counts) < 0 or self.tail_pages == 0:
            raise ValueError("Invalid page policy: page counts must be integers, "
                             "the prefix and suffix >= 0 and the tail ring >= 1")

    @property
    def storage_pages(self) -> int:
        """Exact sidecar pages per admission slot: prefix, suffix, ring."""
        return self.prefix_pages + self.suffix_pages + self.tail_pages


class _Pages:
    """Classification of one request's logical pages at one length."""

    __slots__ = ("policy", "prompt_pages", "pages", "suffix_begin", "ring_begin")

    def __init__(self, policy: Policy, prompt_tokens: int, current_tokens: int) -> None:
        if (type(prompt_tokens) is not int or type(current_tokens) is not int
                or prompt_tokens <= 0 or current_tokens < prompt_tokens):
            raise ValueError("Invalid prompt/current length: need 0 < prompt <= current")
        self.policy = policy
        self.prompt_pages = prompt_tokens // PAGE              # whole prompt pages
        self.pages = -(-current_tokens // PAGE)                # pages holding tokens
        self.suffix_begin = self.prompt_pages - policy.suffix_pages
        self.ring_begin = self.pages - policy.tail_pages
        if self.suffix_begin < policy.prefix_pages or self.ring_begin <= policy.prefix_pages:
            raise ValueError("Prompt cannot support this policy (too few pages for its exact "
                             "prefix and suffix); serve it with the FP16 cache")

    def is_exact(self, page: int) -> bool:
        return (page < self.policy.prefix_pages
                or self.suffix_begin <= page < self.prompt_pages
                or page >= self.ring_begin)

    def history(self) -> tuple:
        return tuple(p for p in range(self.pages) if not self.is_exact(p))


def partition(prompt_tokens: int, current_tokens: int, policy: Policy = Policy()) -> dict:
    """Split a request's pages at ``current_tokens`` into the exact prefix,
    static suffix and tail ring (which may overlap) and the INT8 history,
    every page exactly once (the reference's partition,
    experiments/mlsys2027/serving_v1/pagegauge_vllm/partition.py:23-40).  The
    newest page (possibly partial) is always in the ring, never history."""
    view = _Pages(policy, prompt_tokens, current_tokens)
    history = view.history()
    if not history:
        raise ValueError("Prompt cannot support this policy: no INT8 history page")
    prefix = tuple(range(policy.prefix_pages))
    suffix = tuple(range(view.suffix_begin, view.prompt_pages))
    tail = tuple(range(view.ring_begin, view.pages))
    exact = tuple(p for p in range(view.pages) if view.is_exact(p))
    last_tokens = current_tokens - (view.pages - 1) * PAGE
    return {"prefix": prefix, "suffix": suffix, "tail": tail, "exact": exact,
            "history": history, "history_tokens": PAGE * len(history),
            "exact_tokens": current_tokens - PAGE * len(history),
            "tail_tokens": (policy.tail_pages - 1) * PAGE + last_tokens}


def exact_slot(logical_page: int, prompt_tokens: int, lease_slot: int,
               policy: Policy = Policy()) -> int:
    """Exact sidecar page of ``logical_page`` for the request in admission
    slot ``lease_slot``.  Each slot owns ``policy.storage_pages`` consecutive
    sidecar pages laid out [prefix | suffix | ring]; ring pages rotate by
    logical page modulo the ring length (partition.py:43-52)."""
    if logical_page < 0 or lease_slot < 0:
        raise ValueError("Negative page/lease slot")
    prompt_pages = prompt_tokens // PAGE
    suffix_begin = prompt_pages - policy.suffix_pages
    base = lease_slot * policy.storage_pages
    if logical_page < policy.prefix_pages:
        return base + logical_page
    if suffix_begin <= logical_page < prompt_pages:
        return base + policy.prefix_pages + (logical_page - suffix_begin)
    return base + policy.prefix_pages + policy.suffix_pages + logical_page % policy.tail_pages


# ---------------------------------------------------------------------------
# The ledger: admission slots as state machines + page ownership
# ---------------------------------------------------------------------------

class Phase(enum.Enum):
    FREE = "free"
    PREFILL = "prefill"        # admitted; its prefill is being computed and packed
    PACKING = "packing"        # every layer packed; waiting for the packing event
    READY = "ready"            # decodable
    RETIRING = "retiring"      # finished; waiting for its last-use event


class Lease(NamedTuple):
    """A request's claim on an admission slot; the generation distinguishes
    successive occupants of one slot (centers and sidecars are per slot)."""

    request_id: str
    slot: int
    generation: int


class RequestView(NamedTuple):
    """Immutable view of one admitted request."""

    lease: Lease
    prompt_tokens: int
    current_tokens: int
    physical_pages: tuple


@dataclass
class _Slot:
    generation: int = 0
    phase: Phase = Phase.FREE
    request_id: Optional[str] = None
    prompt_tokens: int = 0
    current_tokens: int = 0
    pages: tuple = ()
    event: Any = None
    stamp: int = 0             # bumped on every change of this slot


def _require_event(event) -> None:
    if not callable(getattr(event, "query", None)):
        raise ValueError("A recorded completion event (an object with query()) is required")


@dataclass(frozen=True)
class StepRow:
    """One scheduled request of a staged decode step."""

    lease: Lease
    prompt_tokens: int
    position: int                   # the token this step appends
    physical_pages: tuple           # block table covering position + 1 tokens
    physical_token_slot: int        # physical page * 16 + row of the token
    exact_token_slot: int           # exact sidecar page * 16 + row of the token
    aged_pages: tuple               # logical pages that become INT8 history
    aged_physical_pages: tuple
    aged_exact_slots: tuple         # the sidecar pages they leave
    stamp: int = 0                  # the slot's stamp when staged

    @property
    def new_history_logical_pages(self) -> tuple:
        return self.aged_pages


@dataclass(frozen=True)
class DecodeStep:
    """A validated decode step, rows in the engine's row order."""

    rows: tuple

    def columns(self) -> dict:
        """Integer columns of the step, one entry per row."""
        return {"request_slots": tuple(r.lease.slot for r in self.rows),
                "generations": tuple(r.lease.generation for r in self.rows),
                "positions": tuple(r.position for r in self.rows),
                "physical_token_slots": tuple(r.physical_token_slot for r in self.rows),
                "exact_token_slots": tuple(r.exact_token_slot for r in self.rows)}


class Ledger:
    """Every admission slot of a served cache and the pool's page ownership.

    ``capacity`` slots (each with its exact sidecar and centers);
    ``pool_pages`` bounds the physical page ids when given.  ``num_layers``
    is the number of layers a prefill must pack before its request becomes
    decodable (``mark_packed``); ``admit(..., ready=True)`` skips the packing
    phases for callers that pack synchronously."""

    def __init__(self, capacity: int, policy: Policy = Policy(), num_layers: int = 1,
                 pool_pages: Optional[int] = None) -> None:
        if type(capacity) is not int or capacity < 1:
            raise ValueError("Positive fixed admission capacity required")
        if type(num_layers) is not int or num_layers < 1:
            raise ValueError("Positive layer count required")
        if pool_pages is not None and (type(pool_pages) is not int or pool_pages < 1):
            raise ValueError("Positive physical pool capacity required")
        self.policy = policy
        self.num_layers = num_layers
        self.pool_pages = pool_pages
        self._slots = [_Slot() for _ in range(capacity)]
        self._slot_of: dict[str, int] = {}
        self._owner: dict[int, int] = {}      # physical page -> slot

    # -- transactions --------------------------------------------------------
    def snapshot(self):
        """Opaque copy of the whole ledger, for ``restore``."""
        return [_Slot(**vars(s)) for s in self._slots], dict(self._slot_of), dict(self._owner)

    def restore(self, snapshot) -> None:
        slots, slot_of, owner = snapshot
        self._slots = [_Slot(**vars(s)) for s in slots]
        self._slot_of, self._owner = dict(slot_of), dict(owner)

    # -- queries -------------------------------------------------------------
    @property
    def capacity(self) -> int:
        return len(self._slots)

    def owner(self, page: int) -> Optional[Lease]:
        """The lease owning physical ``page``, or None."""
        slot = self._owner.get(page)
        return None if slot is None else self._lease(slot)

    def _lease(self, slot: int) -> Lease:
        s = self._slots[slot]
        return Lease(s.request_id, slot, s.generation)

    def _slot(self, lease: Lease) -> _Slot:
        """The live slot of ``lease``; a lease of a previous occupant fails."""
        if not isinstance(lease, Lease) or not 0 <= lease.slot < len(self._slots):
            raise ValueError("Stale request lease: not a lease of this ledger")
        s = self._slots[lease.slot]
        if (s.phase is Phase.FREE or s.generation != lease.generation
                or s.request_id != lease.request_id):
            raise ValueError("Stale request lease: its slot has been reclaimed or reused")
        return s

    def lease_of(self, request_id: str) -> Lease:
        slot = self._slot_of.get(request_id)
        if slot is None:
            raise ValueError(f"Unknown request {request_id!r}")
        return self._lease(slot)

    def view(self, lease: Lease) -> RequestView:
        s = self._slot(lease)
        return RequestView(lease, s.prompt_tokens, s.current_tokens, s.pages)

    def phase(self, lease: Lease) -> Phase:
        return self._slot(lease).phase

    def _table(self, pages, tokens: int) -> tuple:
        """A request's block table for ``tokens`` tokens: one distinct,
        non-negative (in-pool) id per page."""
        table = tuple(pages)
        need = -(-tokens // PAGE)
        if len(table) != need:
            raise ValueError(f"Wrong physical block table: {len(table)} pages for {tokens} "
                             f"tokens (need {need})")
        bad = [p for p in table if type(p) is not int or p < 0
               or (self.pool_pages is not None and p >= self.pool_pages)]
        if bad or len(set(table)) != len(table):
            raise ValueError("Wrong physical block table: ids must be distinct in-pool integers")
        return table

    # -- admission and lifecycle ---------------------------------------------
    def admit(self, request_id: str, prompt_tokens: int, physical_pages, *,
              ready: bool = False) -> Lease:
        """Reserve the lowest free slot for a request with a complete
        ``prompt_tokens`` prefill in ``physical_pages``."""
        if not isinstance(request_id, str) or not request_id:
            raise ValueError("Invalid request ID")
        if request_id in self._slot_of:
            raise ValueError(f"Request {request_id!r} is a duplicate live request")
        partition(prompt_tokens, prompt_tokens, self.policy)
        table = self._table(physical_pages, prompt_tokens)
        if any(p in self._owner for p in table):
            raise ValueError("A prompt page belongs to a live request (no page sharing)")
        free = next((i for i, s in enumerate(self._slots) if s.phase is Phase.FREE), None)
        if free is None:
            raise MemoryError("Declared admission capacity (exact sidecar slots) reached")
        s = self._slots[free]
        s.generation += 1
        s.phase = Phase.READY if ready else Phase.PREFILL
        s.request_id, s.prompt_tokens, s.current_tokens, s.pages = (
            request_id, prompt_tokens, prompt_tokens, table)
        s.event = None
        s.stamp += 1
        self._slot_of[request_id] = free
        for page in table:
            self._owner[page] = free
        return self._lease(free)

    def mark_packed(self, lease: Lease, packed_layers, completion_event) -> None:
        """Every layer of the lease's prefill has been packed into the cache;
        it becomes decodable once ``completion_event`` has fired."""
        s = self._slot(lease)
        if s.phase is not Phase.PREFILL:
            raise ValueError(f"Packing already submitted (lease is {s.phase.value})")
        layers = tuple(packed_layers)
        if any(type(i) is not int for i in layers) or sorted(layers) != list(range(self.num_layers)):
            raise ValueError("Every layer must be packed exactly once")
        _require_event(completion_event)
        s.phase, s.event = Phase.PACKING, completion_event
        s.stamp += 1

    def is_ready(self, lease: Lease) -> bool:
        """Whether the lease is decodable (a fired packing event promotes it)."""
        s = self._slot(lease)
        if s.phase is Phase.PACKING and s.event.query():
            s.phase, s.event = Phase.READY, None
            s.stamp += 1
        return s.phase is Phase.READY

    def retire(self, lease: Lease, last_use_event) -> None:
        """The request has finished (or aborted); its slot and pages return
        to the pool by ``reclaim`` once ``last_use_event`` has fired."""
        s = self._slot(lease)
        if s.phase is Phase.RETIRING:
            raise ValueError("Lease already retiring")
        _require_event(last_use_event)
        s.phase, s.event = Phase.RETIRING, last_use_event
        s.stamp += 1

    def reclaim(self, lease: Lease) -> bool:
        """Free a retiring lease whose last-use event has fired; False while
        its device work is still pending."""
        s = self._slot(lease)
        if s.phase is not Phase.RETIRING:
            raise ValueError("Reclaiming needs an explicit finish/abort (retire) first")
        if not s.event.query():
            return False
        self._free(lease.slot)
        return True

    def release(self, lease: Lease) -> None:
        """Free a lease at once (its device work is known to be over)."""
        self._slot(lease)
        self._free(lease.slot)

    def _free(self, slot: int) -> None:
        s = self._slots[slot]
        for page in s.pages:
            if self._owner.get(page) != slot:
                raise RuntimeError("Page ownership table is corrupted")
            del self._owner[page]
        del self._slot_of[s.request_id]
        self._slots[slot] = _Slot(generation=s.generation, stamp=s.stamp + 1)

    # -- decode steps ----------------------------------------------------------
    def stage_decode(self, scheduled) -> DecodeStep:
        """Validate one decode step without changing the ledger.

        ``scheduled``: (lease, position, block table) per row, in the engine's
        row order; ``position`` must be the request's next token and the block
        table must extend the request's pages (pages it adds must be free and
        distinct across the step)."""
        rows, seen, claimed = [], set(), set()
        for lease, position, physical_pages in scheduled:
            s = self._slot(lease)
            if s.phase is not Phase.READY and not self.is_ready(lease):
                raise RuntimeError(f"Request {lease.request_id!r} is not decodable "
                                   f"({s.phase.value})")
            if lease.request_id in seen:
                raise ValueError("Duplicate scheduled request in one step")
            seen.add(lease.request_id)
            if type(position) is not int or position != s.current_tokens:
                raise ValueError(f"Wrong next token position {position} for a request of "
                                 f"{s.current_tokens} tokens (skipped or replayed token)")
            table = self._table(physical_pages, position + 1)
            if table[:len(s.pages)] != s.pages:
                raise ValueError("Preemption/remapping of existing pages is not supported")
            for page in table[len(s.pages):]:
                if page in self._owner:
                    raise ValueError(f"New physical page {page} belongs to a live request")
                if page in claimed:
                    raise ValueError(f"Physical page {page} aliased across the step's rows")
                claimed.add(page)
            before = _Pages(self.policy, s.prompt_tokens, position)
            after = _Pages(self.policy, s.prompt_tokens, position + 1)
            aged = tuple(p for p in range(after.pages)
                         if before.is_exact(p) and not after.is_exact(p))
            if any((p + 1) * PAGE > position + 1 for p in aged):
                raise RuntimeError("An unfinished page would become INT8 history")
            page, row = divmod(position, PAGE)
            rows.append(StepRow(
                lease, s.prompt_tokens, position, table, table[page] * PAGE + row,
                exact_slot(page, s.prompt_tokens, lease.slot, self.policy) * PAGE + row,
                aged, tuple(table[p] for p in aged),
                tuple(exact_slot(p, s.prompt_tokens, lease.slot, self.policy) for p in aged),
                s.stamp))
        return DecodeStep(tuple(rows))

    def commit_decode(self, step: DecodeStep) -> tuple:
        """Apply a staged step after the caller has fenced its GPU work: each
        row's request grows by one token and owns its new pages.  Nothing
        changes unless every row is still current (its slot unchanged since
        staging, its new pages still free)."""
        if not isinstance(step, DecodeStep):
            raise ValueError("Not a staged decode step")
        for row in step.rows:
            s = self._slot(row.lease)
            if s.stamp != row.stamp or s.phase is not Phase.READY:
                raise ValueError("Decode step is stale: a request changed after staging")
            if any(page in self._owner for page in row.physical_pages[len(s.pages):]):
                raise ValueError("Decode step is stale: a new page was claimed after staging")
        for row in step.rows:
            s = self._slots[row.lease.slot]
            for page in row.physical_pages[len(s.pages):]:
                self._owner[page] = row.lease.slot
            s.current_tokens = row.position + 1
            s.pages = row.physical_pages
            s.stamp += 1
        return tuple({"lease": r.lease, "position": r.position,
                      "closed_page": r.position // PAGE if (r.position + 1) % PAGE == 0 else None,
                      "new_history_pages": r.aged_pages} for r in step.rows)


# ---------------------------------------------------------------------------
# Device tables of one step (K2 scatter ids, K1 CSR tables)
# ---------------------------------------------------------------------------

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


def decode_tables(step: DecodeStep, policy: Policy, device="cuda") -> DecodeTables:
    """The K2 ids and K1 tables of a staged step, for the context after each
    row's token is appended (position + 1 tokens)."""
    import torch

    positions, exact_ids, code_ids, slots = [], [], [], []
    old_ptr, old_idx, exact_ptr, exact_idx, exact_last = [0], [], [0], [], []
    for row in step.rows:
        prompt = row.prompt_tokens
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
    rows = len(step.rows)
    return DecodeTables(t(positions), t(exact_ids), t(code_ids), t(slots), t(old_ptr), t(old_idx),
                        t([PAGE] * rows), t(exact_ptr), t(exact_idx), t(exact_last))


# ---------------------------------------------------------------------------
# Pool geometry, sidecars and zero-copy pool views
# ---------------------------------------------------------------------------

def _plane_specs(pages: int, kv_heads: int, head_dim: int = 128):
    """(name, dtype name, shape) of the four planes of one layer's page pool,
    in storage order: K codes, V codes, K scales, V scales."""
    codes = (pages, PAGE, kv_heads, head_dim)
    scales = (pages, kv_heads)
    return (("key_codes", "int8", codes), ("value_codes", "int8", codes),
            ("key_scales", "float16", scales), ("value_scales", "float16", scales))


def _nbytes(dtype_name: str, shape) -> int:
    count = 1
    for extent in shape:
        count *= extent
    return count * (1 if dtype_name == "int8" else 2)


@dataclass(frozen=True)
class Layout:
    """Geometry of one served cache: ``layers`` layers of a pool of
    ``physical_pages`` INT8 pages (codes + scales), and for each of
    ``maximum_requests`` admission slots an exact FP16 sidecar of
    ``policy.storage_pages`` pages plus its K/V centers and output center
    (the reference's cache_layout.py interface)."""

    layers: int
    physical_pages: int
    maximum_requests: int
    kv_heads: int = 8
    query_heads: int = 32
    head_dim: int = 128
    policy: Policy = Policy()

    def __post_init__(self) -> None:
        dims = (self.layers, self.physical_pages, self.maximum_requests, self.kv_heads,
                self.query_heads, self.head_dim)
        if not all(type(d) is int and d > 0 for d in dims) or self.query_heads % self.kv_heads:
            raise ValueError("Invalid cache geometry: positive integers, query heads a "
                             "multiple of KV heads")

    def sidecar_shapes(self) -> dict:
        exact = (self.layers, self.maximum_requests * self.policy.storage_pages, PAGE,
                 self.kv_heads, self.head_dim)
        center = (self.layers, self.maximum_requests, self.kv_heads, self.head_dim)
        return {"exact_key": exact, "exact_value": exact, "key_center": center,
                "value_center": center,
                "output_center": (self.layers, self.maximum_requests, self.query_heads,
                                  self.head_dim)}

    def accounting(self) -> dict:
        """Bytes of every persistent tensor of the served cache."""
        pool = {name: self.layers * _nbytes(dtype, shape)
                for name, dtype, shape in _plane_specs(self.physical_pages, self.kv_heads,
                                                       self.head_dim)}
        sidecars = {name: _nbytes("float16", shape) for name, shape in self.sidecar_shapes().items()}
        per_page = sum(_nbytes(dtype, shape)
                       for _, dtype, shape in _plane_specs(1, self.kv_heads, self.head_dim))
        return {"tensors": {**pool, **sidecars},
                "page_pool_bytes": sum(pool.values()),
                "reserved_sidecar_bytes": sum(sidecars.values()),
                "total_served_capacity_bytes": sum(pool.values()) + sum(sidecars.values()),
                "per_layer_page_bytes": per_page}

    def admissible_pages(self, cache_budget_bytes: int) -> int:
        """Physical pages a byte budget holds once every sidecar is reserved."""
        acc = self.accounting()
        left = cache_budget_bytes - acc["reserved_sidecar_bytes"]
        if left < 0:
            raise MemoryError("Budget cannot hold the reserved exact/center sidecars")
        return left // (self.layers * acc["per_layer_page_bytes"])


def allocate_sidecars(layout: Layout, *, device, cache_budget_bytes: int) -> dict:
    """Zeroed exact pages and centers of every admission slot, after
    checking that the pool and all sidecars fit ``cache_budget_bytes``."""
    import torch

    if type(cache_budget_bytes) is not int or cache_budget_bytes < 0:
        raise ValueError("Nonnegative integer cache-only byte budget required")
    acc = layout.accounting()
    if acc["total_served_capacity_bytes"] > cache_budget_bytes:
        raise MemoryError("The code pool plus every reserved sidecar exceeds the cache budget")
    tensors = {name: torch.zeros(shape, dtype=torch.float16, device=device)
               for name, shape in layout.sidecar_shapes().items()}
    if sum(t.numel() * 2 for t in tensors.values()) != acc["reserved_sidecar_bytes"]:
        raise RuntimeError("Sidecar allocation differs from the declared accounting")
    return tensors


def dense_pool_views(raw, physical_pages: int, kv_heads: int, head_dim: int = 128) -> dict:
    """The four planes of one layer's pool carved out of one contiguous uint8
    allocation, without a copy, in the layouts K1 and K2 read: codes
    [pages, 16, Hkv, 128] int8 and scales [pages, Hkv] fp16."""
    import torch

    if not all(type(x) is int and x > 0 for x in (physical_pages, kv_heads, head_dim)):
        raise ValueError("Positive integer pool geometry required")
    specs = _plane_specs(physical_pages, kv_heads, head_dim)
    total = sum(_nbytes(dtype, shape) for _, dtype, shape in specs)
    if (raw.dtype != torch.uint8 or raw.dim() != 1 or not raw.is_contiguous()
            or raw.numel() != total or raw.data_ptr() % 16):
        raise ValueError("A 16-byte aligned, contiguous uint8 allocation of exactly "
                         f"{total} bytes is required")
    views, offset = {}, 0
    for name, dtype, shape in specs:
        size = _nbytes(dtype, shape)
        views[name] = raw[offset:offset + size].view(getattr(torch, dtype)).view(shape)
        offset += size
    return views


def from_engine_layer(layer, physical_pages: int, kv_heads: int) -> dict:
    """``dense_pool_views`` of one layer of a packed engine cache whose pages
    are [Hkv, 1, 2*16*128 + 4] uint8 (codes of K and V, then the two fp16
    scales, per head), reinterpreted in place."""
    import torch

    shape = (physical_pages, kv_heads, 1, 2 * PAGE * 128 + 4)
    if layer.dtype != torch.uint8 or tuple(layer.shape) != shape or not layer.is_contiguous():
        raise ValueError("A compact packed engine layer is required; copying is forbidden")
    return dense_pool_views(layer.view(-1), physical_pages, kv_heads)


def zero_physical_pages(views: dict, page_ids) -> None:
    """Clear fresh pages in all four planes (one index fill per plane on the
    current stream) before they are written; nothing changes if any id is
    invalid."""
    import torch

    planes = [views[name] for name, _, _ in _plane_specs(1, 1)]
    pages = tuple(page_ids)
    count = planes[0].shape[0]
    if any(p.shape[0] != count or p.device != planes[0].device for p in planes):
        raise ValueError("Inconsistent pool views")
    if (any(type(p) is not int or not 0 <= p < count for p in pages)
            or len(set(pages)) != len(pages)):
        raise ValueError("Page ids to zero must be distinct, in-pool integers")
    if pages:
        index = torch.tensor(pages, dtype=torch.int64, device=planes[0].device)
        for plane in planes:
            plane.index_fill_(0, index, 0)
