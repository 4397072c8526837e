"""Scheduler messages -> PageGauge admissions, packing and decode steps.

Drop-in for the reference prototype's bridge interface
(experiments/mlsys2027/serving_v1/test_pinned_scheduler_bridge.py:47-175):
``SchedulerBridge(maximum_requests, num_layers, num_physical_pages)`` with
``apply(output, request_order=, last_use_events=)``, ``complete(step,
packed_layers, event)``, ``abort(step, event)``, ``state(request_id)`` and
``PendingDeviceWork``.  A message is vLLM's ``SchedulerOutput`` (duck-typed
on its field names; vLLM is not a dependency here).

Design: the bridge is a thin transaction layer over one ``serving.Ledger``
(the per-slot state machine and page-ownership table).  ``apply`` first
checks everything that depends only on the message (unsupported features,
request shapes, token counts, row order), then performs the message's
effects on the ledger in order -- retire and reclaim finished requests, check
the pages to zero, admit the new requests, stage one decode token per cached
request -- under a snapshot that is restored if any step fails, so a rejected
message leaves no trace.  One step is in flight at a time; ``complete``
marks its prefills packed and commits its decode rows once the caller's event
covers its GPU work, and ``abort`` retires every request of a failed step.
This module never touches the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass

from .serving import PAGE, DecodeStep, Lease, Ledger, Policy, RequestView

# SchedulerOutput fields of features this cache does not serve; a message
# with any of them set (truthy) is rejected before it has any effect.
UNSUPPORTED_FIELDS = (
    "scheduled_spec_decode_tokens", "scheduled_encoder_inputs", "free_encoder_mm_hashes",
    "preempted_req_ids", "num_invalid_spec_tokens", "kv_connector_metadata",
    "has_sync_kv_loads", "ec_connector_metadata", "ec_manager_metadata",
    "kv_cache_block_copies", "kv_connector_block_state", "num_spec_tokens_to_schedule",
)


class PendingDeviceWork(RuntimeError):
    """A finished request's last GPU use has not completed yet: nothing was
    applied; offer the same message again later."""


@dataclass(frozen=True)
class SchedulerStep:
    request_ids: tuple        # the engine's request-row order
    prefills: tuple           # RequestView of every newly admitted request, in row order
    decode: DecodeStep        # staged decode rows, in row order
    zero_pages: tuple         # fresh physical pages the engine must clear first


def _check_message(output) -> list:
    """Everything about a message that does not depend on the cache state;
    returns the scheduled request ids (new requests, then cached ones)."""
    for name in UNSUPPORTED_FIELDS:
        if getattr(output, name, None):
            raise ValueError(f"Unsupported scheduler feature: {name}")
    if any(output.num_common_prefix_blocks or ()):
        raise ValueError("Prefix sharing is unsupported")
    cached = output.scheduled_cached_reqs
    if cached.resumed_req_ids or cached.new_token_ids:
        raise ValueError("Preemption/resume and pipeline-parallel token ids are unsupported")
    columns = (cached.new_block_ids, cached.num_computed_tokens, cached.num_output_tokens)
    if any(len(column) != len(cached.req_ids) for column in columns):
        raise ValueError("Cached-request columns have different lengths")
    for request in output.scheduled_new_reqs:
        if (request.prompt_token_ids is None or request.prompt_embeds is not None
                or request.mm_features or request.lora_request is not None
                or request.pooling_params is not None or request.prefill_token_ids is not None
                or (request.prompt_is_token_ids is not None
                    and not all(request.prompt_is_token_ids))):
            raise ValueError("Only text-token, non-LoRA generation is supported")
        if request.num_computed_tokens != 0:
            raise ValueError("Prefix reuse / chunked prefill is unsupported")
    ids = [r.req_id for r in output.scheduled_new_reqs] + list(cached.req_ids)
    if len(set(ids)) != len(ids):
        raise ValueError("A request is scheduled twice (or both new and cached)")
    counts = output.num_scheduled_tokens
    if (set(counts) != set(ids) or any(type(c) is not int or c < 1 for c in counts.values())
            or sum(counts.values()) != output.total_num_scheduled_tokens):
        raise ValueError("Scheduled token counts do not match the scheduled requests")
    for request in output.scheduled_new_reqs:
        if counts[request.req_id] != len(request.prompt_token_ids):
            raise ValueError("A new request must prefill its whole prompt in one step")
    for name in cached.req_ids:
        if counts[name] != 1:
            raise ValueError("Exactly one decode token per cached request is supported")
        if name in output.finished_req_ids:
            raise ValueError(f"Request {name!r} is both finished and scheduled")
    return ids


class SchedulerBridge:
    """One served cache driven by scheduler messages (one step in flight)."""

    def __init__(self, maximum_requests: int, num_layers: int, num_physical_pages: int,
                 policy: Policy = Policy()) -> None:
        self.ledger = Ledger(maximum_requests, policy, num_layers, num_physical_pages)
        self._pending: SchedulerStep | None = None

    def state(self, request_id: str) -> RequestView:
        return self.ledger.view(self.ledger.lease_of(request_id))

    def _block_table(self, groups) -> tuple:
        groups = tuple(groups)
        if len(groups) != 1:
            raise ValueError("Exactly one KV-cache group is supported")
        return tuple(groups[0])

    def apply(self, output, *, request_order=None, last_use_events=None) -> SchedulerStep:
        """Validate and install one scheduler message as a whole, or change
        nothing.  ``request_order``: the engine's actual row order (default:
        new requests, then cached ones).  ``last_use_events``: the Lease of
        every known finished request -> the event after its last GPU use."""
        if self._pending is not None:
            raise RuntimeError("The previous scheduler step is still in flight")
        ids = _check_message(output)
        order = tuple(ids if request_order is None else request_order)
        if sorted(order) != sorted(ids):
            raise ValueError("The request-row order must list each scheduled request once")
        ledger = self.ledger
        snapshot = ledger.snapshot()
        try:
            step = self._install(output, order, dict(last_use_events or {}))
        except BaseException:
            ledger.restore(snapshot)
            raise
        self._pending = step
        return step

    def _install(self, output, order, events) -> SchedulerStep:
        ledger = self.ledger
        finished = []
        for name in sorted(output.finished_req_ids):
            try:
                finished.append(ledger.lease_of(name))
            except ValueError:
                continue                            # never admitted here: nothing to free
        if set(events) != set(finished):
            raise ValueError("Give exactly one last-use event per known finished request")
        for lease in finished:
            ledger.retire(lease, events[lease])
            if not ledger.reclaim(lease):
                raise PendingDeviceWork(f"Finished request {lease.request_id!r} still has "
                                        "device work in flight")
        zero = tuple(output.new_block_ids_to_zero or ())
        if len(set(zero)) != len(zero) or any(
                type(p) is not int or not 0 <= p < ledger.pool_pages for p in zero):
            raise ValueError("Pages to zero must be distinct in-pool page ids")
        if any(ledger.owner(p) is not None for p in zero):
            raise ValueError("Zeroing would destroy a live request's cache")
        prefills = {}
        for request in output.scheduled_new_reqs:
            lease = ledger.admit(request.req_id, len(request.prompt_token_ids),
                                 self._block_table(request.block_ids))
            prefills[request.req_id] = ledger.view(lease)
        cached = output.scheduled_cached_reqs
        rows = {}
        for name, position, blocks in zip(cached.req_ids, cached.num_computed_tokens,
                                          cached.new_block_ids):
            lease = ledger.lease_of(name)
            table = ledger.view(lease).physical_pages
            if blocks is not None:
                table = table + self._block_table(blocks)
            rows[name] = (lease, position, table)
        decode = ledger.stage_decode([rows[n] for n in order if n in rows])
        return SchedulerStep(order, tuple(prefills[n] for n in order if n in prefills), decode,
                             zero)

    def _check_pending(self, step: SchedulerStep, event) -> bool:
        if step is not self._pending:
            raise ValueError("Unknown, stale or already completed scheduler step")
        if not callable(getattr(event, "query", None)):
            raise ValueError("A recorded completion event (an object with query()) is required")
        return bool(event.query())

    def complete(self, step: SchedulerStep, packed_layers: dict, completion_event) -> bool:
        """Once ``completion_event`` covers the step's GPU work: mark every
        new request packed (``packed_layers[lease]`` lists each layer once)
        and commit the decode rows.  False (nothing changed) while the event
        is pending."""
        if not self._check_pending(step, completion_event):
            return False
        new = {view.lease for view in step.prefills}
        if set(packed_layers) != new:
            raise ValueError("Packed layers must be given for exactly the step's new requests")
        ledger = self.ledger
        snapshot = ledger.snapshot()
        try:
            for lease in sorted(new, key=lambda lease: lease.slot):
                ledger.mark_packed(lease, packed_layers[lease], completion_event)
                ledger.is_ready(lease)
            ledger.commit_decode(step.decode)
        except BaseException:
            ledger.restore(snapshot)
            raise
        self._pending = None
        return True

    def abort(self, step: SchedulerStep, last_use_event) -> bool:
        """Free every request of a failed step once ``last_use_event`` covers
        its device work (the engine aborts them and frees their pages); other
        requests keep their leases."""
        if not self._check_pending(step, last_use_event):
            return False
        ledger = self.ledger
        for name in step.request_ids:
            ledger.release(ledger.lease_of(name))
        self._pending = None
        return True


__all__ = ["PAGE", "UNSUPPORTED_FIELDS", "Lease", "PendingDeviceWork", "SchedulerBridge",
           "SchedulerStep"]
