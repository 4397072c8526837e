"""Page-table algebra against the reference tests' golden lists (CPU).

Golden values come from tests/test_page_gauge_transformer.py:100-216,
:377-427 and :785-870 and tests/test_flashinfer_page_affine_int8.py:50-57 of
the reference; the partition, slot table and exact-table order are also
checked against a page-by-page definition of the page classes over a sweep
of shapes (a static suffix before, inside and behind the tail ring).
"""

from __future__ import annotations

import pytest
import torch

from pagegauge_amd import page_table as pt
from pagegauge_amd.decode import segment_page_table


def test_request_major_page_tables_cover_full_and_ring_storage():
    full = pt.request_major_page_table(2, 4, device="cpu")
    ring = pt.request_major_page_table(2, 4, 2, device="cpu")
    assert full.tolist() == [[0, 1, 2, 3], [4, 5, 6, 7]]
    assert ring.tolist() == [[0, 1, 0, 1], [2, 3, 2, 3]]


def test_exact_sink_partition_is_disjoint_and_covers_context_once():
    partition = pt.page_gauge_logical_partition(total_pages=1283, exact_tail_pages=16,
                                                exact_sink_pages=1, last_page_len=7)
    assert partition["sink_logical_pages"] == (0,)
    assert partition["old_logical_pages"] == tuple(range(1, 1267))
    assert partition["tail_logical_pages"] == tuple(range(1267, 1283))
    assert partition["old_page_count"] == 1266
    assert partition["exact_page_count"] == 17
    assert partition["old_token_count"] == 1266 * pt.PAGE
    assert partition["exact_token_count"] == pt.PAGE + 15 * pt.PAGE + 7
    assert partition["context_token_count"] == 1282 * pt.PAGE + 7
    assert partition["coverage_disjoint"] is True


def test_exact_sink_page_table_uses_slot_zero_then_chronological_tail():
    physical = pt.request_major_exact_page_table(batch_size=2, logical_page_capacity=8,
                                                 exact_tail_pages=2, exact_sink_pages=1,
                                                 device="cpu")
    destination = torch.full((2, 3), -1, dtype=torch.int32)
    active = pt.write_exact_sink_tail_page_table(destination, physical, tail_logical_begin=6,
                                                 total_page_count=8, exact_sink_pages=1)
    assert physical.tolist() == [[0, 2, 1, 2, 1, 2, 1, 2], [3, 5, 4, 5, 4, 5, 4, 5]]
    assert active.tolist() == [[0, 1, 2], [3, 4, 5]]
    assert active.data_ptr() == destination.data_ptr()


def test_exact_prefix_s3_partition_and_page_table_are_disjoint_and_chronological():
    partition = pt.page_gauge_logical_partition(8, 2, 3, pt.PAGE)
    assert partition["prefix_logical_pages"] == (0, 1, 2)
    assert partition["sink_logical_pages"] == (0, 1, 2)
    assert partition["old_logical_pages"] == (3, 4, 5)
    assert partition["tail_logical_pages"] == (6, 7)
    assert partition["coverage_disjoint"] is True
    assert partition["old_token_count"] + partition["exact_token_count"] == \
        partition["context_token_count"]
    physical = pt.request_major_exact_page_table(2, 8, 2, 3, device="cpu")
    destination = torch.full((2, 5), -1, dtype=torch.int32)
    active = pt.write_exact_prefix_tail_page_table(destination, physical, tail_logical_begin=6,
                                                   total_page_count=8, exact_sink_pages=3)
    assert physical.tolist() == [[0, 1, 2, 4, 3, 4, 3, 4], [5, 6, 7, 9, 8, 9, 8, 9]]
    assert active.tolist() == [[0, 1, 2, 3, 4], [5, 6, 7, 8, 9]]


def test_exact_prefix_partition_fails_closed_for_negative_or_no_old_pages():
    with pytest.raises(ValueError, match="nonnegative integer"):
        pt.page_gauge_logical_partition(8, 2, -1, pt.PAGE)
    with pytest.raises(ValueError, match="quantized old page"):
        pt.page_gauge_logical_partition(3, 2, 1, pt.PAGE)
    with pytest.raises(ValueError, match="quantized old page"):
        pt.page_gauge_logical_partition(5, 2, 3, pt.PAGE)
    with pytest.raises(ValueError, match="segmented flashinfer_merge"):
        pt.validate_exact_prefix_attention_path(3, "fused_kernel")
    with pytest.raises(ValueError, match="segmented flashinfer_merge"):
        pt.validate_exact_prefix_attention_path(3, "heterogeneous_fa2")
    assert pt.validate_exact_prefix_attention_path(3, "flashinfer_merge") == 3


def test_heterogeneous_page_table_uses_old_storage_then_exact_ring():
    full = pt.request_major_page_table(2, 5, device="cpu")
    ring = pt.request_major_page_table(2, 5, 2, device="cpu")
    destination = torch.full((2, 5), -1, dtype=torch.int32)
    active = pt.write_heterogeneous_page_table(destination, full, ring, old_page_count=3,
                                               total_page_count=5)
    assert active.tolist() == [[0, 1, 2, 1, 0], [5, 6, 7, 3, 2]]
    assert active.data_ptr() == destination.data_ptr()
    with pytest.raises(ValueError, match="outside table capacity"):
        pt.write_heterogeneous_page_table(destination, full, ring, 4, 6)


def test_segment_page_table_keeps_disjoint_sink_and_tail_exact():
    """tests/test_flashinfer_page_affine_int8.py:50-57."""
    old_indptr, old_indices, exact_indptr, exact_indices = segment_page_table(
        [8, 6], tail_pages=2, sink_pages=1, device="cpu")
    assert old_indptr.tolist() == [0, 5, 8]
    assert old_indices.tolist() == [1, 2, 3, 4, 5, 9, 10, 11]
    assert exact_indptr.tolist() == [0, 3, 6]
    assert exact_indices.tolist() == [0, 6, 7, 8, 12, 13]


@pytest.mark.parametrize("total,tail,sink,last", [
    (17, 16, 0, 1), (257, 16, 1, 16), (40, 3, 5, 9), (3072, 16, 0, 16), (1026, 16, 4, 1)])
def test_partition_covers_every_page_exactly_once(total, tail, sink, last):
    part = pt.page_gauge_logical_partition(total, tail, sink, last)
    pages = part["old_logical_pages"] + part["exact_logical_pages"]
    assert sorted(pages) == list(range(total))
    assert set(part["old_logical_pages"]).isdisjoint(part["exact_logical_pages"])
    assert part["old_token_count"] + part["exact_token_count"] == (total - 1) * 16 + last
    # the tail ring reuses slots: logical pages that share a slot never coexist in the tail
    physical = pt.request_major_exact_page_table(1, total, tail, sink, device="cpu")[0].tolist()
    tail_slots = [physical[p] for p in part["tail_logical_pages"]]
    assert len(set(tail_slots)) == len(tail_slots)
    assert set(tail_slots).isdisjoint(physical[p] for p in part["sink_logical_pages"])


def test_static_suffix_partition_and_table():
    part = pt.page_gauge_logical_partition(20, 4, 1, 5, exact_static_suffix_pages=2,
                                           initial_context_pages=12)
    assert part["static_suffix_logical_pages"] == (10, 11)
    assert part["old_logical_pages"] == tuple(range(1, 10)) + (12, 13, 14, 15)
    physical = pt.request_major_exact_page_table(2, 20, 4, 1, exact_static_suffix_pages=2,
                                                 initial_context_pages=12, device="cpu")
    assert physical[0, 0].item() == 0 and physical[0, 10].item() == 1 and physical[0, 11].item() == 2
    assert physical[1].tolist() == [v + 7 for v in physical[0].tolist()]
    for p in range(20):
        assert pt.exact_physical_page_index(1, p, 4, 1, 2, 12) == physical[1, p].item()
    with pytest.raises(ValueError, match="initial old-cache page"):
        pt.validate_exact_static_suffix_pages(3, exact_prefix_pages=2, initial_context_pages=5)


def test_flatten_page_table():
    table = pt.request_major_page_table(3, 4, device="cpu")
    indptr, indices = pt.flatten_page_table(table, [4, 0, 2])
    assert indptr.tolist() == [0, 4, 4, 6]
    assert indices.tolist() == [0, 1, 2, 3, 8, 9]
    with pytest.raises(ValueError, match="outside the table"):
        pt.flatten_page_table(table, [5, 0, 0])


def test_old_page_table_writer_rejects_unsorted_sets():
    full = pt.request_major_page_table(1, 6, device="cpu")
    destination = torch.full((1, 6), -1, dtype=torch.int32)
    active = pt.write_page_gauge_old_page_table(destination, full, (1, 2, 4))
    assert active.tolist() == [[1, 2, 4]]
    with pytest.raises(ValueError, match="unique and increasing"):
        pt.write_page_gauge_old_page_table(destination, full, (2, 1))


def test_fixed_suffix_mapping_and_partition_are_exact_once():
    """tests/test_page_gauge_transformer.py:785-824 of the reference."""
    prefix, suffix, tail, initial = 4, 64, 48, 1280
    storage = prefix + suffix + tail
    assert pt.exact_physical_page_index(0, 0, tail, prefix, suffix, initial) == 0
    assert pt.exact_physical_page_index(0, initial - suffix, tail, prefix, suffix, initial) == prefix
    assert pt.exact_physical_page_index(0, initial - 1, tail, prefix, suffix,
                                        initial) == prefix + suffix - 1
    generated = initial
    assert pt.exact_physical_page_index(0, generated, tail, prefix, suffix,
                                        initial) == prefix + suffix + generated % tail
    assert pt.exact_physical_page_index(1, generated, tail, prefix, suffix,
                                        initial) == storage + prefix + suffix + generated % tail
    first = pt.page_gauge_logical_partition(initial, tail, prefix, pt.PAGE, suffix, initial)
    assert first["exact_page_count"] == prefix + suffix
    assert first["old_logical_pages"] == tuple(range(prefix, initial - suffix))
    assert first["coverage_disjoint"]
    later = pt.page_gauge_logical_partition(initial + tail, tail, prefix, 13, suffix, initial)
    assert later["exact_page_count"] == prefix + suffix + tail
    assert set(later["old_logical_pages"]).isdisjoint(later["static_suffix_logical_pages"])
    assert later["coverage_disjoint"]


def test_fixed_suffix_active_tables_are_unique_and_keep_current_page_last():
    """tests/test_page_gauge_transformer.py:827-870 of the reference."""
    prefix, suffix, tail, initial = 4, 64, 48, 1280
    logical = pt.request_major_exact_page_table(1, initial + 96, tail, prefix, suffix, initial,
                                                device="cpu")
    destination = torch.empty(1, prefix + suffix + tail, dtype=torch.int32)
    first = pt.write_exact_prefix_tail_page_table(destination, logical, initial - tail, initial,
                                                  prefix, suffix, initial)
    assert first.shape[1] == prefix + suffix
    assert len(set(first[0].tolist())) == prefix + suffix
    nxt = pt.write_exact_prefix_tail_page_table(destination, logical, initial - tail + 1,
                                                initial + 1, prefix, suffix, initial)
    assert nxt.shape[1] == prefix + suffix + 1
    assert len(set(nxt[0].tolist())) == prefix + suffix + 1
    assert nxt[0, -1].item() == pt.exact_physical_page_index(0, initial, tail, prefix, suffix,
                                                             initial)


def test_decoder_style_fixed_suffix_tables():
    """The tables of the reference's fixed-suffix decoder plan
    (tests/test_page_gauge_transformer.py:377-427): capacity 10, tail 2,
    prefix 1, suffix 2, initial context 8 pages, at 8 and 9 pages."""
    full = pt.request_major_page_table(1, 10, device="cpu")
    exact = pt.request_major_exact_page_table(1, 10, 2, 1, 2, 8, device="cpu")
    old_dst = torch.empty(1, 10, dtype=torch.int32)
    exact_dst = torch.empty(1, 5, dtype=torch.int32)
    for pages, want_old, want_exact in ((8, [1, 2, 3, 4, 5], [0, 1, 2]),
                                        (9, [1, 2, 3, 4, 5], [0, 1, 2, 3])):
        part = pt.page_gauge_logical_partition(pages, 2, 1, 1 if pages == 9 else pt.PAGE, 2, 8)
        old = pt.write_page_gauge_old_page_table(old_dst, full, part["old_logical_pages"])
        ex = pt.write_exact_prefix_tail_page_table(exact_dst, exact, part["tail_logical_begin"],
                                                   pages, 1, 2, 8)
        assert old.tolist() == [want_old]
        assert ex.tolist() == [want_exact]
        assert part["old_page_count"] + part["exact_page_count"] == pages


def _classify(page, total, tail, prefix, suffix, initial):
    """Definition of the page classes, one page at a time."""
    if page < prefix:
        return "exact"
    if suffix and initial - suffix <= page < initial:
        return "exact"
    if page >= total - tail:
        return "exact"
    return "old"


@pytest.mark.parametrize("total,tail,prefix,suffix,initial", [
    (20, 4, 1, 2, 12), (12, 4, 1, 2, 12), (13, 4, 1, 2, 12), (14, 4, 0, 3, 12),
    (40, 3, 5, 0, None), (1300, 48, 4, 64, 1280), (1290, 48, 4, 64, 1280),
    (30, 16, 2, 5, 25), (60, 16, 2, 5, 25)])
def test_partition_tables_match_the_page_by_page_definition(total, tail, prefix, suffix, initial):
    """Old/exact sets, slot table and exact-table order against the page-class
    definition above, including a tail ring that still overlaps the suffix."""
    part = pt.page_gauge_logical_partition(total, tail, prefix, 5, suffix, initial)
    want_old = [p for p in range(total) if _classify(p, total, tail, prefix, suffix, initial) == "old"]
    assert list(part["old_logical_pages"]) == want_old
    assert list(part["exact_logical_pages"]) == [p for p in range(total) if p not in set(want_old)]
    assert part["old_token_count"] == 16 * len(want_old)
    assert part["exact_token_count"] == (total - 1) * 16 + 5 - 16 * len(want_old)
    # slots: prefix fixed, suffix fixed after it, everything else on the ring
    capacity = total + 7
    table = pt.request_major_exact_page_table(3, capacity, tail, prefix, suffix, initial,
                                              device="cpu")
    storage = prefix + suffix + tail
    for r in range(3):
        for p in range(capacity):
            if p < prefix:
                want = p
            elif suffix and initial - suffix <= p < initial:
                want = prefix + p - (initial - suffix)
            else:
                want = prefix + suffix + p % tail
            assert table[r, p].item() == r * storage + want
            assert pt.exact_physical_page_index(r, p, tail, prefix, suffix, initial) == r * storage + want
    # the exact table lists every exact page of the context once, on distinct slots
    dst = torch.full((1, storage + 4), -1, dtype=torch.int32)
    active = pt.write_exact_prefix_tail_page_table(dst, table[:1], part["tail_logical_begin"], total,
                                                   prefix, suffix, initial)[0].tolist()
    listed = list(range(prefix)) + (list(range(initial - suffix, initial)) if suffix else [])
    listed += [p for p in range(total - tail, total) if p not in listed]
    assert active == [table[0, p].item() for p in listed]
    assert len(set(active)) == len(active)
    exact_now = set(part["exact_logical_pages"])
    assert exact_now <= set(listed)


@pytest.mark.parametrize("call,match", [
    (lambda: pt.exact_physical_page_index(-1, 0, 4), "non-negative with a tail"),
    (lambda: pt.exact_physical_page_index(0, 0, 0), "non-negative with a tail"),
    (lambda: pt.request_major_exact_page_table(1, 4, 2, 4, device="cpu"), "smaller than logical"),
    (lambda: pt.request_major_exact_page_table(0, 4, 2, device="cpu"), "must be positive"),
    (lambda: pt.request_major_page_table(1, 4, 0, device="cpu"), "physical pages per request"),
    (lambda: pt.page_gauge_logical_partition(8, 2, 1, 0), "outside one page"),
    (lambda: pt.page_gauge_logical_partition(8, 0, 1, 3), "must be positive"),
    (lambda: pt.validate_exact_static_suffix_pages(2), "positive initial context"),
    (lambda: pt.validate_exact_static_suffix_pages(-1), "nonnegative integer"),
    (lambda: pt.validate_exact_sink_pages(2), "0 or 1"),
])
def test_page_table_messages(call, match):
    with pytest.raises(ValueError, match=match):
        call()


def test_table_writers_reject_bad_tables():
    good = torch.zeros(2, 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="exact page tables must use int32"):
        pt.write_exact_prefix_tail_page_table(good.long(), good, 6, 8, 1)
    with pytest.raises(ValueError, match="exact page tables must have shape"):
        pt.write_exact_prefix_tail_page_table(good[0], good, 6, 8, 1)
    with pytest.raises(ValueError, match="exact page-table batch sizes differ"):
        pt.write_exact_prefix_tail_page_table(good[:1], good, 6, 8, 1)
    with pytest.raises(ValueError, match="overlap or are empty"):
        pt.write_exact_prefix_tail_page_table(good, good, 8, 8, 1)
    with pytest.raises(ValueError, match="exceeds allocated capacity"):
        pt.write_exact_prefix_tail_page_table(good, good, 6, 9, 1)
    with pytest.raises(ValueError, match="exceeds destination capacity"):
        pt.write_exact_prefix_tail_page_table(good[:, :2], good, 5, 8, 1)
    with pytest.raises(ValueError, match="old page tables must use int32"):
        pt.write_page_gauge_old_page_table(good, good.long(), (1,))
    with pytest.raises(ValueError, match="old page set cannot be empty"):
        pt.write_page_gauge_old_page_table(good, good, ())
    with pytest.raises(ValueError, match="old logical page exceeds"):
        pt.write_page_gauge_old_page_table(good, good, (1, 8))
    with pytest.raises(ValueError, match="exceeds destination capacity"):
        pt.write_page_gauge_old_page_table(good[:, :1], good, (1, 2))
    with pytest.raises(ValueError, match="matching"):
        pt.write_heterogeneous_page_table(good, good[:1], good, 1, 2)
