"""Page-table algebra against the reference tests' golden lists (CPU).

Golden values come from tests/test_page_gauge_transformer.py:100-216 and
tests/test_flashinfer_page_affine_int8.py:50-57 of the reference; the
exact-once partition invariants are checked over a sweep of shapes.
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
