"""Request lifecycle and scheduler transactions of a served PageGauge cache.

Host restatement of the reference's serving prototype
(experiments/mlsys2027/serving_v1/pagegauge_vllm/prefill_lifecycle.py:10-97,
scheduler_bridge.py:13-215), with the same rules and messages:

* ``PrefillLifecycle``: a lease is reserved at admission, becomes decodable
  only once every layer has been packed (prefill population) and the caller's
  completion event has fired, and is reclaimed only after its last-use event.
* ``SchedulerBridge``: one scheduler message (vLLM's ``SchedulerOutput``
  fields, duck-typed: vLLM is not a dependency) is validated as a whole
  transaction on a copy of the bookkeeping (retirements, zeroed pages,
  one-shot prefills, one decode token per cached request) and only then
  installed; ``complete`` / ``abort`` advance or roll back after the caller's
  event covers the step's GPU work.

Events are any objects with ``query()`` (``torch.cuda.Event`` is one); this
module never touches the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass

from .serving import DecodeBatch, Lease, Policy, RequestSlots, commit_decode, prepare_decode

PREFILL, PACKING, READY, RETIRING = "prefill", "packing", "ready", "retiring"


def _require_event(event) -> None:
    if not callable(getattr(event, "query", None)):
        raise ValueError("A recorded completion event is required")


class PrefillLifecycle:
    """Phases of each lease: prefill -> packing -> ready -> retiring
    (prefill_lifecycle.py:10-97)."""

    def __init__(self, maximum_requests: int, num_layers: int, policy: Policy = Policy()) -> None:
        if type(num_layers) is not int or num_layers < 1:
            raise ValueError("Positive layer count required")
        self.num_layers = num_layers
        self.slots = RequestSlots(maximum_requests, policy)
        self._phase: dict[Lease, str] = {}
        self._event: dict[Lease, object] = {}

    def clone(self) -> "PrefillLifecycle":
        other = PrefillLifecycle.__new__(PrefillLifecycle)
        other.num_layers = self.num_layers
        other.slots = self.slots.clone()
        other._phase = dict(self._phase)
        other._event = dict(self._event)
        return other

    def begin(self, request_id: str, prompt_tokens: int, block_groups,
              num_computed_tokens: int = 0) -> Lease:
        """Reserve a slot for a one-shot prefill; not decodable yet."""
        if num_computed_tokens != 0:
            raise ValueError("Prefix reuse/chunked prefill is unsupported")
        groups = tuple(block_groups)
        if len(groups) != 1:
            raise ValueError("Exactly one cache group required")
        lease = self.slots.admit(request_id, prompt_tokens, groups[0])
        self._phase[lease] = PREFILL
        return lease

    def submit_packing(self, lease: Lease, packed_layers, completion_event) -> None:
        self.slots.state(lease)
        if self._phase[lease] != PREFILL:
            raise ValueError("Packing already submitted or lease retiring")
        layers = tuple(packed_layers)
        if any(type(i) is not int for i in layers) or sorted(layers) != list(range(self.num_layers)):
            raise ValueError("Every layer must be packed exactly once")
        _require_event(completion_event)
        self._event[lease] = completion_event
        self._phase[lease] = PACKING

    def ready(self, lease: Lease) -> bool:
        self.slots.state(lease)
        if self._phase[lease] == PACKING and self._event[lease].query():
            self._phase[lease] = READY
            del self._event[lease]
        return self._phase[lease] == READY

    def decode_batch(self, request_ids) -> tuple:
        leases = self.slots.batch(request_ids)
        if not all(self.ready(lease) for lease in leases):
            raise RuntimeError("Decode requested before packing completion or after finish")
        return tuple(self.slots.state(lease) for lease in leases)

    def retire(self, lease: Lease, last_use_event) -> None:
        self.slots.state(lease)
        if self._phase[lease] == RETIRING:
            raise ValueError("Lease already retiring")
        _require_event(last_use_event)
        self._event[lease] = last_use_event
        self._phase[lease] = RETIRING

    def prepare_decode(self, scheduled) -> DecodeBatch:
        scheduled = tuple(scheduled)
        if not all(self.ready(lease) for lease, _, _ in scheduled):
            raise RuntimeError("All decode leases must be ready")
        return prepare_decode(self.slots, scheduled)

    def commit_decode(self, batch: DecodeBatch, completion_event):
        """None while the event is pending; the appended rows once it has fired."""
        _require_event(completion_event)
        if not all(self.ready(row.lease) for row in batch.rows):
            raise RuntimeError("Cannot commit a non-ready or retiring lease")
        if not completion_event.query():
            return None
        return commit_decode(self.slots, batch)

    def reclaim(self, lease: Lease) -> bool:
        self.slots.state(lease)
        if self._phase[lease] != RETIRING:
            raise ValueError("Explicit finish/abort event required")
        if not self._event[lease].query():
            return False
        self.slots.release(lease)
        del self._event[lease]
        del self._phase[lease]
        return True


class PendingDeviceWork(RuntimeError):
    """A finished lease's last use has not completed; retry the same message later."""


@dataclass(frozen=True)
class SchedulerStep:
    request_ids: tuple        # the engine's request-row order
    prefills: tuple           # State of every newly admitted request, in row order
    decode: DecodeBatch       # validated decode rows, in row order
    zero_pages: tuple         # fresh physical pages the engine must clear first


# SchedulerOutput fields whose features this cache does not support
# (scheduler_bridge.py:69-80); any truthy value rejects the message.
UNSUPPORTED_FIELDS = (
    "scheduled_spec_decode_tokens", "scheduled_encoder_inputs", "free_encoder_mm_hashes",
    "preempted_req_ids", "num_invalid_spec_tokens", "kv_connector_metadata",
    "has_sync_kv_loads", "ec_connector_metadata", "ec_manager_metadata",
    "kv_cache_block_copies", "kv_connector_block_state", "num_spec_tokens_to_schedule",
)


class SchedulerBridge:
    """Scheduler messages -> PageGauge admissions, packing and decode rows
    (scheduler_bridge.py:38-215).  One step is in flight at a time."""

    def __init__(self, maximum_requests: int, num_layers: int, num_physical_pages: int,
                 policy: Policy = Policy()) -> None:
        if type(num_physical_pages) is not int or num_physical_pages < 1:
            raise ValueError("Positive physical pool capacity required")
        self.num_physical_pages = num_physical_pages
        self._lifecycle = PrefillLifecycle(maximum_requests, num_layers, policy)
        self._leases: dict[str, Lease] = {}
        self._pending: SchedulerStep | None = None

    def state(self, request_id: str):
        if request_id not in self._leases:
            raise ValueError("Unknown request")
        return self._lifecycle.slots.state(self._leases[request_id])

    def _pool_pages(self, pages) -> tuple:
        pages = tuple(pages)
        if (len(set(pages)) != len(pages)
                or any(type(p) is not int or not 0 <= p < self.num_physical_pages for p in pages)):
            raise ValueError("Invalid/duplicate physical pool page")
        return pages

    def _one_group(self, groups) -> tuple:
        groups = tuple(groups)
        if len(groups) != 1:
            raise ValueError("Exactly one cache group required")
        return self._pool_pages(groups[0])

    @staticmethod
    def _request_ids(output) -> list:
        """Reject what the cache cannot serve; the scheduled request ids."""
        for name in UNSUPPORTED_FIELDS:
            if getattr(output, name):
                raise ValueError(f"Unsupported scheduler feature: {name}")
        if any(output.num_common_prefix_blocks):
            raise ValueError("Prefix sharing is unsupported")
        cached = output.scheduled_cached_reqs
        if cached.resumed_req_ids or cached.new_token_ids:
            raise ValueError("Preemption/resume and pipeline parallelism unsupported")
        n = len(cached.req_ids)
        if any(len(column) != n for column in (cached.new_block_ids, cached.num_computed_tokens,
                                               cached.num_output_tokens)):
            raise ValueError("Mismatched cached-request columns")
        ids = [r.req_id for r in output.scheduled_new_reqs] + list(cached.req_ids)
        if len(set(ids)) != len(ids):
            raise ValueError("Duplicate/new-and-cached scheduled request")
        counts = output.num_scheduled_tokens
        if (set(counts) != set(ids) or any(type(c) is not int or c < 1 for c in counts.values())
                or sum(counts.values()) != output.total_num_scheduled_tokens):
            raise ValueError("Inconsistent scheduled token counts")
        return ids

    @staticmethod
    def _text_generation(request) -> None:
        if (request.prompt_token_ids is None or request.prompt_embeds is not None
                or request.mm_features or request.lora_request is not None
                or request.pooling_params is not None or request.prefill_token_ids is not None
                or (request.prompt_is_token_ids is not None
                    and not all(request.prompt_is_token_ids))):
            raise ValueError("Only text-token, non-LoRA generation is supported")

    def apply(self, output, *, request_order=None, last_use_events=None) -> SchedulerStep:
        """Validate one scheduler message completely, then install it.

        ``request_order`` is the engine's actual row order (default: new
        requests, then cached ones).  ``last_use_events`` maps the Lease of
        every known finished request to the event after its last GPU use.
        Nothing changes if any check fails."""
        if self._pending is not None:
            raise RuntimeError("Previous scheduler step is still in flight")
        ids = self._request_ids(output)
        order = tuple(ids if request_order is None else request_order)
        if len(order) != len(ids) or set(order) != set(ids):
            raise ValueError("Actual request-row order must cover each request once")
        trial = self._lifecycle.clone()
        leases = dict(self._leases)
        events = dict(last_use_events or {})
        finished = {leases[name] for name in output.finished_req_ids if name in leases}
        if set(events) != finished:
            raise ValueError("Supply one last-use event per known finished lease")
        for lease in sorted(finished, key=lambda lease: lease.slot):
            trial.retire(lease, events[lease])
            if not trial.reclaim(lease):
                raise PendingDeviceWork("Finished lease still has outstanding device work")
            del leases[lease.request_id]

        zero_pages = self._pool_pages(output.new_block_ids_to_zero or ())
        if any(p in trial.slots.page_owner for p in zero_pages):
            raise ValueError("Zeroing would destroy a live request cache")

        prefills = {}
        for request in output.scheduled_new_reqs:
            self._text_generation(request)
            length = len(request.prompt_token_ids)
            if output.num_scheduled_tokens[request.req_id] != length:
                raise ValueError("One-shot complete prefill required; no chunking")
            pages = self._one_group(request.block_ids)
            lease = trial.begin(request.req_id, length, (pages,), request.num_computed_tokens)
            leases[request.req_id] = lease
            prefills[request.req_id] = trial.slots.state(lease)

        cached = output.scheduled_cached_reqs
        decode_rows = {}
        for i, name in enumerate(cached.req_ids):
            if name not in leases or name in output.finished_req_ids:
                raise ValueError("Unknown or finished cached request")
            if output.num_scheduled_tokens[name] != 1:
                raise ValueError("Exactly one decode token per cached request required")
            lease = leases[name]
            pages = trial.slots.state(lease).physical_pages
            if cached.new_block_ids[i] is not None:
                pages = pages + self._one_group(cached.new_block_ids[i])
            self._pool_pages(pages)
            decode_rows[name] = (lease, cached.num_computed_tokens[i], pages)
        batch = trial.prepare_decode([decode_rows[n] for n in order if n in decode_rows])
        step = SchedulerStep(order, tuple(prefills[n] for n in order if n in prefills), batch,
                             zero_pages)
        self._lifecycle, self._leases, self._pending = trial, leases, step
        return step

    def _fired(self, step: SchedulerStep, event) -> bool:
        if step is not self._pending:
            raise ValueError("Unknown, stale or already completed scheduler step")
        _require_event(event)
        return bool(event.query())

    def complete(self, step: SchedulerStep, packed_layers: dict, completion_event) -> bool:
        """Commit the step's prefills (every layer packed) and decode rows once
        ``completion_event`` covers its GPU work; False (nothing advanced)
        while it is pending."""
        if not self._fired(step, completion_event):
            return False
        if set(packed_layers) != {state.lease for state in step.prefills}:
            raise ValueError("Packing coverage must match exactly the new leases")
        trial = self._lifecycle.clone()
        for state in step.prefills:
            trial.submit_packing(state.lease, packed_layers[state.lease], completion_event)
            if not trial.ready(state.lease):
                return False
        if trial.commit_decode(step.decode, completion_event) is None:
            return False
        self._lifecycle, self._pending = trial, None
        return True

    def abort(self, step: SchedulerStep, last_use_event) -> bool:
        """Reclaim every request of a failed step once its device work has
        ended; the engine aborts them and frees their physical pages."""
        if not self._fired(step, last_use_event):
            return False
        trial = self._lifecycle.clone()
        leases = dict(self._leases)
        for name in step.request_ids:
            lease = leases.pop(name)
            trial.retire(lease, last_use_event)
            if not trial.reclaim(lease):
                return False
        self._lifecycle, self._leases, self._pending = trial, leases, None
        return True
