"""Serving metadata on the CPU: the S/A/T partition, exact slots, the
ledger's slot state machine and page ownership, staged decode steps, device
tables and pool accounting.

Expectations follow the reference's serving prototype
(experiments/mlsys2027/serving_v1/pagegauge_vllm/, pinned by
test_pinned_scheduler_bridge.py: 4096-token prompts of 256 pages, the first
decode token's physical slot 512*16 when block 512 is appended)."""

from __future__ import annotations

import pytest
import torch

from pagegauge_amd import serving as sv

PAGE = 16


def test_default_policy_partition_of_a_4096_token_prompt():
    part = sv.partition(4096, 4096)
    assert part["prefix"] == (0, 1, 2, 3)
    assert part["suffix"] == tuple(range(128, 256))
    assert part["tail"] == tuple(range(208, 256))
    assert part["history"] == tuple(range(4, 128))
    assert part["history_tokens"] == 124 * 16 and part["exact_tokens"] == 4096 - 124 * 16
    assert part["tail_tokens"] == 48 * 16
    # the first decode token opens page 256; the tail moves, the suffix stays
    nxt = sv.partition(4096, 4097)
    assert nxt["tail"] == tuple(range(209, 257)) and nxt["history"] == part["history"]
    assert nxt["tail_tokens"] == 47 * 16 + 1


@pytest.mark.parametrize("prompt,current", [(4096, 4096), (4100, 4200), (3000, 5000), (2500, 2500)])
def test_partition_covers_every_page_exactly_once(prompt, current):
    part = sv.partition(prompt, current)
    pages = (current + 15) // 16
    assert sorted(part["history"] + part["exact"]) == list(range(pages))
    assert not set(part["history"]) & set(part["exact"])
    assert pages - 1 in part["exact"]                      # the open page is never history
    assert part["history_tokens"] + part["exact_tokens"] == current


@pytest.mark.parametrize("args,message", [
    ((0, 16), "Invalid prompt/current length"),
    ((100, 50), "Invalid prompt/current length"),
    ((1024, 1024), "Prompt cannot support this policy"),      # 64 pages < 4 + 128
])
def test_partition_errors(args, message):
    with pytest.raises(ValueError, match=message):
        sv.partition(*args)


def test_policy_validation_and_storage():
    with pytest.raises(ValueError, match="Invalid page policy"):
        sv.Policy(tail_pages=0)
    with pytest.raises(ValueError, match="Invalid page policy"):
        sv.Policy(prefix_pages=-1)
    assert sv.Policy().storage_pages == 180


def test_exact_slot_layout():
    pol = sv.Policy()
    assert sv.exact_slot(2, 4096, 3, pol) == 3 * 180 + 2                 # prefix
    assert sv.exact_slot(130, 4096, 3, pol) == 3 * 180 + 4 + 2           # static suffix
    assert sv.exact_slot(300, 4096, 3, pol) == 3 * 180 + 132 + 300 % 48  # tail ring
    with pytest.raises(ValueError, match="Negative page/lease slot"):
        sv.exact_slot(-1, 4096, 0, pol)


def _append(ledger, lease, position, table):
    """Stage and commit one token of one request."""
    return ledger.commit_decode(ledger.stage_decode([(lease, position, table)]))[0]


def test_ledger_slots_and_generations():
    ledger = sv.Ledger(2)
    a = ledger.admit("a", 4096, range(256), ready=True)
    b = ledger.admit("b", 4096, range(256, 512), ready=True)
    assert (a.slot, a.generation, b.slot) == (0, 1, 1)
    with pytest.raises(MemoryError, match="admission capacity"):
        ledger.admit("c", 4096, range(512, 768))
    with pytest.raises(ValueError, match="duplicate live request"):
        ledger.admit("a", 4096, range(800, 1056))
    info = _append(ledger, a, 4096, list(range(256)) + [900])
    assert info["closed_page"] is None and info["new_history_pages"] == ()
    assert ledger.owner(900) == a
    with pytest.raises(ValueError, match="skipped or replayed token"):
        _append(ledger, a, 4096, list(range(256)) + [900])
    with pytest.raises(ValueError, match="New physical page 900 belongs to a live request"):
        _append(ledger, b, 4096, list(range(256, 512)) + [900])
    with pytest.raises(ValueError, match="remapping"):
        _append(ledger, b, 4096, list(range(257, 513)) + [901])
    ledger.release(a)
    assert ledger.owner(900) is None and ledger.owner(0) is None
    with pytest.raises(ValueError, match="Stale request lease"):
        ledger.view(a)
    again = ledger.admit("a", 4096, range(256))
    assert (again.slot, again.generation) == (0, 2)        # the slot is reused, generation bumped
    with pytest.raises(ValueError, match="Wrong physical block table"):
        ledger.admit("d", 4096, [0] * 256)
    with pytest.raises(ValueError, match="Wrong physical block table"):
        sv.Ledger(1, pool_pages=100).admit("e", 4096, range(256))   # ids beyond the pool


def test_pages_age_into_history_only_when_complete():
    ledger = sv.Ledger(1, sv.Policy(prefix_pages=1, suffix_pages=2, tail_pages=2))
    lease = ledger.admit("a", 160, range(10), ready=True)   # 10 pages; history 1..6
    table = list(range(10))
    aged = []
    for position in range(160, 160 + 40):
        if position % 16 == 0:
            table.append(100 + position // 16)
        info = _append(ledger, lease, position, table)
        aged.extend(info["new_history_pages"])
        for page in info["new_history_pages"]:
            assert page < (position + 1) // 16             # only completed pages
    # prompt pages 8, 9 are the static suffix (exact for good); page 10 left
    # the 2-page tail ring when page 12 opened (position 192)
    assert aged == [10]


def test_staged_decode_steps_match_the_reference_bridge():
    ledger = sv.Ledger(3)
    a = ledger.admit("a", 4096, range(256), ready=True)
    step = ledger.stage_decode([(a, 4096, list(range(256)) + [512])])
    row = step.rows[0]
    assert row.physical_token_slot == 512 * 16                 # test_pinned_scheduler_bridge.py:61
    assert row.exact_token_slot == sv.exact_slot(256, 4096, a.slot) * 16
    assert step.columns()["positions"] == (4096,)
    assert ledger.view(a).current_tokens == 4096               # staging changes nothing
    assert ledger.owner(512) is None
    ledger.commit_decode(step)
    assert ledger.view(a).current_tokens == 4097 and ledger.owner(512) == a
    with pytest.raises(ValueError, match="Decode step is stale"):
        ledger.commit_decode(step)
    with pytest.raises(ValueError, match="Wrong next token position"):
        ledger.stage_decode([(a, 4096, list(range(256)) + [512])])
    b = ledger.admit("b", 4096, range(600, 856), ready=True)
    c = ledger.admit("c", 4096, range(900, 1156), ready=True)
    with pytest.raises(ValueError, match="aliased across the step"):
        ledger.stage_decode([(b, 4096, list(range(600, 856)) + [513]),
                             (c, 4096, list(range(900, 1156)) + [513])])
    with pytest.raises(ValueError, match="Duplicate scheduled request"):
        ledger.stage_decode([(b, 4096, list(range(600, 856)) + [2000])] * 2)
    # a page claimed after staging makes the staged step stale
    step_b = ledger.stage_decode([(b, 4096, list(range(600, 856)) + [3000])])
    ledger.commit_decode(ledger.stage_decode([(c, 4096, list(range(900, 1156)) + [3000])]))
    with pytest.raises(ValueError, match="claimed after staging"):
        ledger.commit_decode(step_b)
    assert ledger.view(b).current_tokens == 4096


def test_slot_phases():
    class Event:
        def __init__(self, done):
            self.done = done

        def query(self):
            return self.done

    ledger = sv.Ledger(2, num_layers=3)
    lease = ledger.admit("a", 4096, range(256))
    assert ledger.phase(lease) is sv.Phase.PREFILL
    with pytest.raises(RuntimeError, match="not decodable"):
        ledger.stage_decode([(lease, 4096, list(range(256)) + [300])])
    with pytest.raises(ValueError, match="completion event"):
        ledger.mark_packed(lease, [0, 1, 2], object())
    with pytest.raises(ValueError, match="Every layer must be packed exactly once"):
        ledger.mark_packed(lease, [0, 1], Event(True))
    event = Event(False)
    ledger.mark_packed(lease, [2, 0, 1], event)
    with pytest.raises(ValueError, match="Packing already submitted"):
        ledger.mark_packed(lease, [0, 1, 2], event)
    assert not ledger.is_ready(lease) and ledger.phase(lease) is sv.Phase.PACKING
    event.done = True
    assert ledger.is_ready(lease)
    step = ledger.stage_decode([(lease, 4096, list(range(256)) + [300])])
    assert ledger.commit_decode(step)[0]["position"] == 4096
    with pytest.raises(ValueError, match="retire"):
        ledger.reclaim(lease)
    last = Event(False)
    ledger.retire(lease, last)
    with pytest.raises(ValueError, match="already retiring"):
        ledger.retire(lease, last)
    with pytest.raises(RuntimeError, match="not decodable"):
        ledger.stage_decode([(lease, 4097, list(range(256)) + [300])])
    assert not ledger.reclaim(lease)
    last.done = True
    assert ledger.reclaim(lease) and ledger.owner(300) is None
    with pytest.raises(ValueError, match="Stale request lease"):
        ledger.is_ready(lease)
    with pytest.raises(ValueError, match="Positive layer count"):
        sv.Ledger(1, num_layers=0)


def test_decode_tables_cover_the_context_once():
    pol = sv.Policy(prefix_pages=2, suffix_pages=4, tail_pages=6)
    ledger = sv.Ledger(3, pol)
    leases, tables = [], []
    for name, prompt, base in (("a", 800, 0), ("b", 1000, 100), ("c", 1200, 200)):
        pages = list(range(base, base + (prompt + 15) // 16))
        leases.append(ledger.admit(name, prompt, pages, ready=True))
        tables.append(pages)
    scheduled = []
    for lease, table in zip(leases, tables):
        position = ledger.view(lease).current_tokens
        if position % 16 == 0:
            table = table + [1000 + len(table) + 100 * lease.slot]
        scheduled.append((lease, position, table))
    step = ledger.stage_decode(scheduled)
    t = sv.decode_tables(step, pol, device="cpu")
    for r, (lease, position, table) in enumerate(scheduled):
        prompt = ledger.view(lease).prompt_tokens
        part = sv.partition(prompt, position + 1, pol)
        old = t.old_indices[t.old_indptr[r]:t.old_indptr[r + 1]].tolist()
        exact = t.exact_indices[t.exact_indptr[r]:t.exact_indptr[r + 1]].tolist()
        assert old == [table[p] for p in part["history"]]
        assert exact == [sv.exact_slot(p, prompt, lease.slot, pol) for p in part["exact"]]
        assert exact[-1] == int(t.exact_page_ids[r])               # K2 writes the last exact page
        assert int(t.code_page_ids[r]) == table[position // 16]
        assert len(old) * 16 + (len(exact) - 1) * 16 + int(t.exact_last_page_len[r]) == position + 1
    assert t.positions.dtype == torch.int32 and t.old_last_page_len.tolist() == [16, 16, 16]


def test_layout_accounting():
    layout = sv.Layout(layers=32, physical_pages=1000, maximum_requests=4)
    acc = layout.accounting()
    assert acc["per_layer_page_bytes"] == 2 * 16 * 8 * 128 + 4 * 8
    assert acc["page_pool_bytes"] == 32 * 1000 * (2 * 16 * 8 * 128 + 4 * 8)
    assert acc["tensors"]["exact_key"] == 2 * 32 * 4 * 180 * 16 * 8 * 128
    budget = acc["reserved_sidecar_bytes"] + 10 * 32 * acc["per_layer_page_bytes"]
    assert layout.admissible_pages(budget) == 10
    with pytest.raises(MemoryError):
        layout.admissible_pages(acc["reserved_sidecar_bytes"] - 1)
    with pytest.raises(ValueError, match="Invalid cache geometry"):
        sv.Layout(layers=1, physical_pages=1, maximum_requests=1, query_heads=30)


def test_dense_pool_views_split_one_allocation():
    raw = torch.zeros(2 * 4 * 16 * 8 * 128 + 2 * 4 * 8 * 2, dtype=torch.uint8)
    views = sv.dense_pool_views(raw, 4, 8)
    assert views["key_codes"].shape == (4, 16, 8, 128) and views["value_scales"].shape == (4, 8)
    views["value_scales"].fill_(1.0)
    assert raw[-2:].view(torch.float16).item() == 1.0
    with pytest.raises(ValueError, match="exactly"):
        sv.dense_pool_views(raw[:-2], 4, 8)
