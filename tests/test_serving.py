"""Serving metadata on the CPU: the S/A/T partition, exact slots, request
leases, decode-batch metadata, device tables and pool accounting.

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


def test_request_slot_lifecycle_and_generations():
    slots = sv.RequestSlots(2)
    a = slots.admit("a", 4096, range(256))
    b = slots.admit("b", 4096, range(256, 512))
    assert (a.slot, a.generation, b.slot) == (0, 1, 1)
    with pytest.raises(MemoryError, match="admission capacity"):
        slots.admit("c", 4096, range(512, 768))
    with pytest.raises(ValueError, match="duplicate live request"):
        slots.admit("a", 4096, range(800, 1056))
    info = slots.append(a, 4096, list(range(256)) + [900])
    assert info["closed_page"] is None and info["new_history_pages"] == ()
    with pytest.raises(ValueError, match="Skipped/replayed token"):
        slots.append(a, 4096, list(range(256)) + [900])
    with pytest.raises(ValueError, match="New physical page belongs to a live request"):
        slots.append(b, 4096, list(range(256, 512)) + [900])
    with pytest.raises(ValueError, match="Preemption/remapping"):
        slots.append(b, 4096, list(range(257, 513)) + [901])
    slots.release(a)
    with pytest.raises(ValueError, match="Stale request lease"):
        slots.state(a)
    again = slots.admit("a", 4096, range(256))
    assert (again.slot, again.generation) == (0, 2)        # the slot is reused, generation bumped
    with pytest.raises(ValueError, match="Wrong/duplicate physical block table"):
        slots.admit("d", 4096, [0] * 256)


def test_pages_age_into_history_only_when_complete():
    slots = sv.RequestSlots(1, sv.Policy(prefix_pages=1, suffix_pages=2, tail_pages=2))
    lease = slots.admit("a", 160, range(10))                # 10 pages; history 1..6
    table = list(range(10))
    aged = []
    for position in range(160, 160 + 40):
        if position % 16 == 0:
            table.append(100 + position // 16)
        info = slots.append(lease, position, table)
        aged.extend(info["new_history_pages"])
        for page in info["new_history_pages"]:
            assert page < (position + 1) // 16             # only completed pages
    # prompt pages 8, 9 are the static suffix (exact for good); page 10 left
    # the 2-page tail ring when page 12 opened (position 192)
    assert aged == [10]


def test_prepare_and_commit_decode_match_the_reference_bridge():
    slots = sv.RequestSlots(2)
    a = slots.admit("a", 4096, range(256))
    batch = sv.prepare_decode(slots, [(a, 4096, list(range(256)) + [512])])
    row = batch.rows[0]
    assert row.physical_token_slot == 512 * 16                 # test_pinned_scheduler_bridge.py:66
    assert row.exact_token_slot == sv.exact_slot(256, 4096, a.slot) * 16
    assert batch.columns()["positions"] == (4096,)
    assert slots.state(a).current_tokens == 4096               # non-mutating
    sv.commit_decode(slots, batch)
    assert slots.state(a).current_tokens == 4097
    with pytest.raises(ValueError, match="Decode batch is stale"):
        sv.commit_decode(slots, batch)
    with pytest.raises(ValueError, match="Wrong next token position"):
        sv.prepare_decode(slots, [(a, 4096, list(range(256)) + [512])])
    b = slots.admit("b", 4096, range(600, 856))
    with pytest.raises(ValueError, match="Physical page alias across batch"):
        sv.prepare_decode(slots, [(a, 4097, list(range(256)) + [512]),
                                  (b, 4096, list(range(600, 856)) + [512])])
    with pytest.raises(ValueError, match="Duplicate scheduled request"):
        sv.prepare_decode(slots, [(b, 4096, list(range(600, 856)) + [900])] * 2)


def test_decode_tables_cover_the_context_once():
    pol = sv.Policy(prefix_pages=2, suffix_pages=4, tail_pages=6)
    slots = sv.RequestSlots(3, pol)
    leases, tables = [], []
    for name, prompt, base in (("a", 800, 0), ("b", 1000, 100), ("c", 1200, 200)):
        pages = list(range(base, base + (prompt + 15) // 16))
        leases.append(slots.admit(name, prompt, pages))
        tables.append(pages)
    scheduled = []
    for lease, table in zip(leases, tables):
        position = slots.state(lease).current_tokens
        if position % 16 == 0:
            table = table + [1000 + len(table) + 100 * lease.slot]
        scheduled.append((lease, position, table))
    batch = sv.prepare_decode(slots, scheduled)
    t = sv.decode_tables(batch, pol, device="cpu")
    for r, (lease, position, table) in enumerate(scheduled):
        prompt = slots.state(lease).prompt_tokens
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
    with pytest.raises(ValueError, match="exact size"):
        sv.dense_pool_views(raw[:-2], 4, 8)
