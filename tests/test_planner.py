"""Invariants of the split scheduler (``pg_decode_plan``), checked on the host
through ``pg_decode_plan_host``: every page of every segment is covered by
exactly one work item, items respect the one-lane-per-page cap, a request's
items are contiguous with their FP16 tail first, and the plan fits the
256-CU launch it was balanced for."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from pagegauge_amd import workloads
from pagegauge_amd.decode import plan_work_items

MAX_CHUNK = 64


def _indptr(counts):
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32).tolist()


def _check_cover(items, item_ptr, old_counts, tail_counts):
    batch = len(old_counts)
    items = items.numpy()
    assert (items[:, 4] > items[:, 3]).all(), "empty work item"
    assert (items[:, 4] - items[:, 3] <= MAX_CHUNK).all()
    old_ptr, tail_ptr = _indptr(old_counts), _indptr(tail_counts)
    for b in range(batch):
        mine = items[item_ptr[b]:item_ptr[b + 1]]
        assert (mine[:, 0] == b).all()
        assert list(mine[:, 6]) == list(range(len(mine)))          # item_in_request
        assert (mine[:, 7] == len(mine)).all()                     # items_in_request
        for seg, ptr in ((0, old_ptr), (1, tail_ptr)):
            rows = mine[mine[:, 2] == seg]
            covered = sorted(p for r in rows for p in range(r[3], r[4]))
            assert covered == list(range(ptr[b], ptr[b + 1])), (b, seg)
            if len(rows):
                assert (rows[:, 5] == ptr[b + 1] - 1).all()          # last page of the segment
        if tail_counts[b] and old_counts[b]:
            segs = list(mine[:, 2])
            assert segs == sorted(segs, reverse=True), "tail items come first"


@pytest.mark.parametrize("old,tail", [([3056], [16]), ([240], [16]), ([1], [1]), ([0], [3]),
                                      ([7, 0, 300], [16, 2, 0])])
def test_balanced_plan_covers_every_page_once(old, tail):
    plan, items, ptr = plan_work_items(_indptr(old), [16] * len(old), _indptr(tail),
                                       [16] * len(tail))
    assert plan.num_items == items.shape[0] == ptr[-1]
    assert plan.num_items <= 256 or plan.num_items == sum(
        -(-n // MAX_CHUNK) for n in old + tail)
    _check_cover(items, ptr.tolist(), old, tail)
    assert plan.max_items_per_request == max(int(ptr[b + 1] - ptr[b]) for b in range(len(old)))


@pytest.mark.parametrize("tokens,items,waves", [(4096, 64, 2), (8192, 128, 4), (16400, 112, 4),
                                                (49152, 112, 4), (65536, 112, 4), (114688, 113, 4),
                                                (131072, 256, 8)])
def test_one_request_plan_regimes(tokens, items, waves):
    """Small problems: chunks down to one PV group; medium (3..30 weighted
    pages per CU, B1/49K included): 7/16 of the CUs in items (more only where
    the 64-page item cap needs them), each over two half-height workgroups;
    large (128K tokens: 32 pages per CU): one 8-wave workgroup per item."""
    old = tokens // 16 - 16
    plan, got, _ = plan_work_items([0, old], [16], [0, 16], [16])
    assert (plan.num_items, plan.waves_per_block) == (items, waves)
    assert plan.num_items * (8 // plan.waves_per_block) <= 256      # one wave of workgroups


def test_b8_ragged_plans_stay_large():
    lengths = workloads.ragged_lengths(workloads.VALIDATION_SEEDS[0])
    old = [(n - 256) // 16 for n in lengths]
    plan, items, _ = plan_work_items(_indptr(old), [16] * 8, _indptr([16] * 8), [16] * 8)
    assert plan.waves_per_block == 8 and plan.num_items <= 256
    assert (items[:, 4] - items[:, 3])[items[:, 2] == 0].min() >= 16


def test_b1_49k_plan_uses_sixteen_page_chunks_within_one_wave():
    plan, items, _ = plan_work_items([0, 3056], [16], [0, 16], [16])
    sizes = (items[:, 4] - items[:, 3]).numpy()
    assert plan.num_items <= 256
    old_sizes = sizes[items[:, 2].numpy() == 0]
    assert old_sizes.max() - old_sizes.min() <= 1                  # nearly equal chunks
    assert old_sizes.min() >= 16


@pytest.mark.parametrize("seed", workloads.VALIDATION_SEEDS[:3])
def test_b8_ragged_plan_is_balanced(seed):
    lengths = workloads.ragged_lengths(seed)
    old = [(n - 256) // 16 for n in lengths]
    plan, items, ptr = plan_work_items(_indptr(old), [16] * 8, _indptr([16] * 8), [16] * 8)
    _check_cover(items, ptr.tolist(), old, [16] * 8)
    assert plan.num_items <= 256
    sizes = (items[:, 4] - items[:, 3]).numpy().astype(float)
    weight = np.where(items[:, 2].numpy() == 1, 2.0, 1.0)               # FP16 pages weigh 2x
    load = sizes * weight
    assert load.max() <= 1.25 * np.sort(load)[-len(load) // 4:].mean()


def test_fixed_split_follows_fixed_split_size():
    plan, items, ptr = plan_work_items([0, 100, 130], [16, 5], [0, 16, 20], [16, 16],
                                       split_pages=32)
    _check_cover(items, ptr.tolist(), [100, 30], [16, 4])
    sizes = (items[:, 4] - items[:, 3]).numpy()
    seg = items[:, 2].numpy()
    # ceil(n / split) nearly equal items per segment; tail split defaults to ceil(32/2)
    assert list(sizes[seg == 0]) == [25, 25, 25, 25, 30]
    assert list(sizes[seg == 1]) == [16, 4]
    assert plan.split_pages == 30 and plan.tail_split_pages == 16


def test_fp16_primary_plan_has_no_tail_weighting():
    plan, items, ptr = plan_work_items([0, 512], [16], kv_data_type=torch.float16)
    assert plan.primary_kind == 1 and plan.has_tail == 0
    _check_cover(items, ptr.tolist(), [512], [0])


def test_plan_rejects_too_many_items_per_request():
    with pytest.raises(RuntimeError, match="too many splits"):
        plan_work_items([0, 5000], [16], split_pages=1)



def _closed_form_items(plan, kind):
    """Work items from a plan's closed-form description (the kernel's rule)."""
    rows = []
    for i in range(plan.num_items):
        tail = i < plan.cf_tail_items
        n = plan.cf_tail_pages if tail else plan.cf_primary_pages
        c = plan.cf_tail_items if tail else plan.num_items - plan.cf_tail_items
        k = i if tail else i - plan.cf_tail_items
        base = plan.cf_tail_begin if tail else plan.cf_primary_begin
        q, r = divmod(n, c)
        begin = base + k * q + min(k, r)
        rows.append([0, 1 if tail else kind, int(tail), begin, begin + q + (k < r), base + n - 1,
                     i, plan.num_items, base, 2 if tail and kind == 0 else 1, 0, 0])
    return rows


@pytest.mark.parametrize("old,tail,split,tail_split,dtype", [
    ([0, 3056], [0, 16], 0, 0, torch.int8),          # B1/49K balanced
    ([5, 1014], [3, 19], 0, 0, torch.int8),          # offsets into shared tables
    ([0, 3056], [0, 16], 11, 3, torch.int8),         # fixed splits with remainders
    ([0, 7], [0, 16], 0, 0, torch.int8),
    ([0, 1009], None, 0, 0, torch.float16),          # FP16 pages, no tail
    ([2, 900], None, 5, 0, "heterogeneous"),
    ([0, 0], [0, 16], 0, 0, torch.int8),             # tail only
])
def test_one_request_plans_are_closed_form(old, tail, split, tail_split, dtype):
    plan, items, _ = plan_work_items(old, [16], tail, None if tail is None else [16],
                                     kv_data_type=dtype, split_pages=split,
                                     tail_split_pages=tail_split)
    kind = {torch.int8: 0, torch.float16: 1, "heterogeneous": 2}[dtype]
    assert plan.closed_form == 1
    assert plan.cf_tail_items == plan.num_items - plan.num_items_primary
    assert _closed_form_items(plan, kind) == items.tolist()


def test_batches_keep_the_item_table():
    plan, _, _ = plan_work_items([0, 100, 240], [16, 16], [0, 16, 32], [16, 16])
    assert plan.closed_form == 0
    assert (plan.cf_tail_items, plan.cf_primary_pages) == (0, 0)


@pytest.mark.parametrize("pages,hint", [([1280] * 4, 16), ([37, 5, 900], 16), ([12], 16), ([64], 3)])
def test_heterogeneous_hint_gives_the_ring_its_own_items(pages, hint):
    """exact_tail_pages_hint: the last ``hint`` pages of each unified table
    form items of their own, weighted as FP16 pages; every item keeps the
    request's first and last page, and the table is still covered once."""
    ptr = _indptr(pages)
    plan, items, item_ptr = plan_work_items(ptr, [16] * len(pages), kv_data_type="heterogeneous",
                                            exact_tail_pages_hint=hint)
    _check_cover(items, item_ptr.tolist(), pages, [0] * len(pages))
    it = items.numpy()
    for b, n in enumerate(pages):
        mine = it[it[:, 0] == b]
        assert (mine[:, 8] == ptr[b]).all()                       # request_page_begin
        assert (mine[:, 5] == ptr[b + 1] - 1).all()               # the request's last page
        split = ptr[b + 1] - min(hint, n)
        assert not ((mine[:, 3] < split) & (mine[:, 4] > split)).any()   # no item straddles it
    if pages == [1280] * 4:
        size = it[:, 4] - it[:, 3]
        ring = it[:, 3] >= np.repeat(np.array(ptr[1:]) - hint, [int((it[:, 0] == b).sum())
                                                                 for b in range(4)])
        # FP16 items hold about half the pages of INT8 items (equal weighted load)
        assert size[ring].max() * 2 <= size[~ring].max() + 2


def test_exact_tail_hint_is_checked():
    with pytest.raises(RuntimeError, match="applies to heterogeneous plans"):
        plan_work_items([0, 100], [16], exact_tail_pages_hint=16)
    with pytest.raises(RuntimeError, match="must be non-negative"):
        plan_work_items([0, 100], [16], kv_data_type="heterogeneous", exact_tail_pages_hint=-1)


try:
    from hypothesis import given, settings, strategies as st
except ImportError:                                  # pragma: no cover
    given = None

if given is not None:
    @settings(max_examples=120, deadline=None)
    @given(old=st.lists(st.integers(0, 900), min_size=1, max_size=12),
           tail=st.data(), split=st.sampled_from([None, 1, 3, 4, 16, 64]),
           last=st.data())
    def test_random_batches_cover_every_page_once(old, tail, split, last):
        """Fuzzed batches (empty and one-page segments included): the planner
        covers every INT8 and tail page exactly once, within the 64-page cap,
        with each request's items contiguous, numbered in order and tail
        first, and a workgroup shape that divides the 8 KV heads."""
        tails = tail.draw(st.lists(st.integers(0, 16), min_size=len(old), max_size=len(old)))
        lasts = last.draw(st.lists(st.integers(1, 16), min_size=len(old), max_size=len(old)))
        if sum(old) + sum(tails) == 0:
            return
        plan, items, ptr = plan_work_items(_indptr(old), lasts, _indptr(tails), lasts,
                                           split_pages=split or 0)
        assert plan.num_items == items.shape[0] == ptr[-1]
        _check_cover(items, ptr.tolist(), old, tails)
        assert plan.max_items_per_request == max(int(ptr[b + 1] - ptr[b]) for b in range(len(old)))
        assert plan.waves_per_block in (1, 2, 4, 8) and 8 % plan.waves_per_block == 0


@pytest.mark.parametrize("batch,pages,items", [(16, 1008, 272), (64, 496, 576), (128, 240, 640)])
def test_multi_round_plans_use_four_wave_workgroups(batch, pages, items):
    """More items than CUs: two 4-wave workgroups per CU instead of one
    8-wave workgroup, so that one item's start-up overlaps another's stream;
    plans of at most one item per CU keep their widths (above)."""
    plan, _, _ = plan_work_items(_indptr([pages] * batch), [16] * batch,
                                 _indptr([16] * batch), [16] * batch)
    assert (plan.num_items, plan.waves_per_block) == (items, 4)
