"""Request lifecycle, scheduler transactions and pool views on the CPU.

Cases follow the reference's pinned tests
(experiments/mlsys2027/serving_v1/test_pinned_scheduler_bridge.py:47-175,
test_pinned_cache_spec.py:12-131).  vLLM is not installed, so scheduler
messages are plain namespaces with ``SchedulerOutput``'s field names; events
are fakes with ``query()``."""

from __future__ import annotations

from types import SimpleNamespace
from unittest.mock import patch

import pytest
import torch

from pagegauge_amd import serving as sv
from pagegauge_amd.serving_bridge import UNSUPPORTED_FIELDS, PendingDeviceWork, SchedulerBridge


class Event:
    def __init__(self, done=True):
        self.done = done

    def query(self):
        return self.done


def new_request(name, start=0, prompt=4096):
    return SimpleNamespace(req_id=name, prompt_token_ids=[7] * prompt, mm_features=[],
                           sampling_params=None, pooling_params=None,
                           block_ids=(list(range(start, start + (prompt + 15) // 16)),),
                           num_computed_tokens=0, lora_request=None, prompt_embeds=None,
                           prefill_token_ids=None, prompt_is_token_ids=None)


def message(new=(), cached=(), finished=()):
    out = SimpleNamespace(**{name: None for name in UNSUPPORTED_FIELDS})
    out.num_common_prefix_blocks = []
    out.new_block_ids_to_zero = None
    out.scheduled_new_reqs = list(new)
    out.finished_req_ids = set(finished)
    out.num_scheduled_tokens = {r.req_id: len(r.prompt_token_ids) for r in new}
    data = SimpleNamespace(req_ids=[], resumed_req_ids=set(), new_token_ids=[],
                           new_block_ids=[], num_computed_tokens=[], num_output_tokens=[])
    for name, position, blocks in cached:
        data.req_ids.append(name)
        data.num_computed_tokens.append(position)
        data.num_output_tokens.append(position - 4096 + 1)
        data.new_block_ids.append(None if blocks is None else (list(blocks),))
        out.num_scheduled_tokens[name] = 1
    out.scheduled_cached_reqs = data
    out.total_num_scheduled_tokens = sum(out.num_scheduled_tokens.values())
    return out


@pytest.fixture
def bridge():
    return SchedulerBridge(2, 2, 2048)


def admit(bridge, *requests):
    step = bridge.apply(message(new=requests))
    assert bridge.complete(step, {s.lease: [0, 1] for s in step.prefills}, Event())
    return step


def test_mixed_prefill_and_decode_wait_for_every_layer_and_the_event(bridge):
    admit(bridge, new_request("a"))
    step = bridge.apply(message(new=[new_request("b", 256)], cached=[("a", 4096, [512])]),
                        request_order=["a", "b"])
    assert step.request_ids == ("a", "b")
    assert step.decode.rows[0].physical_token_slot == 512 * 16
    event = Event(False)
    layers = {step.prefills[0].lease: [1, 0]}
    assert not bridge.complete(step, layers, event)
    assert bridge.state("a").current_tokens == 4096
    with pytest.raises(RuntimeError, match="still in flight"):
        bridge.apply(message())
    assert bridge.ledger.phase(step.prefills[0].lease) is sv.Phase.PREFILL
    event.done = True
    with pytest.raises(ValueError, match="Every layer must be packed exactly once"):
        bridge.complete(step, {step.prefills[0].lease: [0]}, event)
    assert bridge.state("a").current_tokens == 4096
    assert bridge.complete(step, layers, event)
    assert bridge.state("a").current_tokens == 4097 and bridge.state("b").current_tokens == 4096
    assert bridge.ledger.phase(bridge.state("b").lease) is sv.Phase.READY
    with pytest.raises(ValueError, match="stale or already completed"):
        bridge.complete(step, layers, event)


def test_unscheduled_rows_keep_their_leases_and_rows_follow_the_engine_order(bridge):
    admit(bridge, new_request("a"), new_request("b", 256))
    a, b = bridge.state("a").lease, bridge.state("b").lease
    bridge.complete(bridge.apply(message(cached=[("b", 4096, [512])])), {}, Event())
    assert bridge.state("a").lease == a
    step = bridge.apply(message(cached=[("a", 4096, [513]), ("b", 4097, None)]),
                        request_order=["b", "a"])
    assert [r.lease for r in step.decode.rows] == [b, a]
    assert step.decode.rows[0].physical_pages[-1] == 512
    bridge.complete(step, {}, Event())
    assert bridge.state("b").current_tokens == 4098


def test_reusing_an_id_waits_for_the_old_lease_and_bumps_the_generation(bridge):
    admit(bridge, new_request("a"))
    old = bridge.state("a").lease
    msg = message(new=[new_request("a")], finished=["a"])
    event = Event(False)
    with pytest.raises(PendingDeviceWork):
        bridge.apply(msg, last_use_events={old: event})
    assert bridge.state("a").lease == old
    event.done = True
    replacement = bridge.apply(msg, last_use_events={old: event}).prefills[0].lease
    assert (replacement.slot, replacement.generation) == (old.slot, old.generation + 1)


def test_a_rejected_message_neither_admits_nor_releases(bridge):
    admit(bridge, new_request("a"))
    old = bridge.state("a").lease
    msg = message(new=[new_request("a"), new_request("b")], finished=["a"])   # b aliases a's pages
    with pytest.raises(ValueError):
        bridge.apply(msg, last_use_events={old: Event()})
    assert bridge.state("a").lease == old
    with pytest.raises(ValueError, match="Unknown request"):
        bridge.state("b")
    assert bridge.apply(message(new=[new_request("b", 256)])).prefills[0].lease.generation == 1


@pytest.mark.parametrize("field,value", [("kv_cache_block_copies", [object()]),
                                         ("preempted_req_ids", {"a"}),
                                         ("scheduled_spec_decode_tokens", {"a": [1]}),
                                         ("num_common_prefix_blocks", [1]),
                                         ("kv_connector_metadata", object())])
def test_unsupported_scheduler_features_are_rejected_before_admission(bridge, field, value):
    msg = message(new=[new_request("a")])
    setattr(msg, field, value)
    with pytest.raises(ValueError):
        bridge.apply(msg)
    assert admit(bridge, new_request("a")).prefills[0].lease.generation == 1


@pytest.mark.parametrize("mode", ["chunk", "reuse", "groups", "resumed", "order", "lora"])
def test_unsupported_request_shapes_are_rejected(bridge, mode):
    request = new_request("a")
    msg = message(new=[request])
    kwargs = {}
    if mode == "chunk":
        msg.num_scheduled_tokens["a"] -= 1
        msg.total_num_scheduled_tokens -= 1
    elif mode == "reuse":
        request.num_computed_tokens = 16
    elif mode == "groups":
        request.block_ids += (list(range(256)),)
    elif mode == "resumed":
        msg.scheduled_cached_reqs.resumed_req_ids = {"a"}
    elif mode == "lora":
        request.lora_request = object()
    else:
        kwargs["request_order"] = ["unknown"]
    with pytest.raises(ValueError):
        bridge.apply(msg, **kwargs)
    assert admit(bridge, new_request("a")).prefills[0].lease.generation == 1


def test_zeroed_pages_cannot_destroy_a_live_cache(bridge):
    admit(bridge, new_request("a"))
    msg = message(cached=[("a", 4096, [256])])
    for pages in ([0], [256, 256], [-1], [2048]):
        msg.new_block_ids_to_zero = pages
        with pytest.raises(ValueError):
            bridge.apply(msg)
    msg.new_block_ids_to_zero = [256]
    assert bridge.apply(msg).zero_pages == (256,)


def test_abort_reclaims_only_the_scheduled_leases_after_the_fence(bridge):
    admit(bridge, new_request("a"), new_request("b", 256))
    b = bridge.state("b").lease
    step = bridge.apply(message(cached=[("a", 4096, [512])]))
    event = Event(False)
    assert not bridge.abort(step, event)
    assert bridge.state("a").current_tokens == 4096
    event.done = True
    assert bridge.abort(step, event)
    with pytest.raises(ValueError):
        bridge.state("a")
    assert bridge.state("b").lease == b


def test_bridge_never_initialises_the_gpu():
    assert not torch.cuda.is_initialized()


def test_sidecars_match_the_declared_accounting():
    layout = sv.Layout(2, 32, 3, kv_heads=1, query_heads=2, policy=sv.Policy(1, 1, 2))
    acc = layout.accounting()
    tensors = sv.allocate_sidecars(layout, device="cpu",
                                   cache_budget_bytes=acc["total_served_capacity_bytes"])
    assert sum(t.untyped_storage().nbytes() for t in tensors.values()) == acc["reserved_sidecar_bytes"]
    assert tensors["exact_key"].shape == (2, 12, 16, 1, 128)
    assert tensors["output_center"].shape == (2, 3, 2, 128)
    assert all(t.dtype == torch.float16 and t.is_contiguous() and not t.count_nonzero()
               for t in tensors.values())
    minimum = sv.Layout(1, 32, 1).accounting()["total_served_capacity_bytes"]
    with patch("torch.zeros") as allocate:
        for budget in (minimum - 1, 0):
            with pytest.raises(MemoryError):
                sv.allocate_sidecars(sv.Layout(1, 32, 1), device="cpu", cache_budget_bytes=budget)
        for budget in (-1, True, float(minimum)):
            with pytest.raises(ValueError):
                sv.allocate_sidecars(sv.Layout(1, 32, 1), device="cpu", cache_budget_bytes=budget)
        allocate.assert_not_called()


def test_engine_layer_views_keep_their_offset_and_zeroing_keeps_other_pages():
    backing = torch.zeros((2, 3, 8, 1, 4100), dtype=torch.uint8)
    views = sv.from_engine_layer(backing[1], 3, 8)
    assert views["key_codes"].data_ptr() == backing[1].data_ptr()
    for t in views.values():
        t.fill_(1)
    assert not backing[0].any() and backing[1].any()
    with pytest.raises(ValueError, match="compact packed engine layer"):
        sv.from_engine_layer(torch.zeros((3, 2, 8, 1, 4100), dtype=torch.uint8)[:, 0], 3, 8)
    raw = torch.empty(4 * 32800, dtype=torch.uint8)
    views = sv.dense_pool_views(raw, 4, 8)
    for t in views.values():
        t.fill_(7)
    sv.zero_physical_pages(views, [3, 1])
    for t in views.values():
        assert (t[[1, 3]] == 0).all() and (t[[0, 2]] == 7).all()
    before = raw.clone()
    for pages in ([0, 4], [0, -1], [0, 0], [True]):
        with pytest.raises(ValueError):
            sv.zero_physical_pages(views, pages)
        assert torch.equal(raw, before)
