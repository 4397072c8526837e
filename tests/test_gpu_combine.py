"""The two combine kernels return the same bits for the same partials.

Plans with at most 32 work items per request and at least 512 (request,
query head) rows merge them with one wave per row (8, 16 or 32 item slots);
other plans use four workgroups per row.  A request planned alone (32 rows:
the four-workgroup kernel) and as the first of 16 requests (512 rows, the
others of 4 items: the row kernel), with the same fixed splits so that its
partials are the same, must give bit-identical out and lse, at item counts
on both sides of each slot size."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import fp16_parity, max_abs, oracle_decode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("pages,split", [(2, 1), (7, 1), (16, 2), (60, 4), (64, 4), (124, 4)])
def test_row_and_block_combines_agree(cuda, pages, split):
    from pagegauge_amd import decode, workloads

    items = -(-pages // split) + 1        # INT8 items + one tail item (tail split 16)
    print(f"combine kernels: {pages} pages / split {split} = {items} items", flush=True)
    lengths = [16 * (16 + pages)] + [16 * (16 + 3 * split)] * 15
    w = workloads.build_decode_workload(lengths, 20261220 + pages, device=cuda, tail_tokens=256)
    w.tail_last_page_len = torch.tensor([11] + [16] * 15, dtype=torch.int32, device=cuda)
    ws = torch.empty(32 << 20, dtype=torch.uint8, device=cuda)
    results = []
    for batch in (1, 16):
        n_old, n_tail = int(w.old_indptr[batch]), int(w.tail_indptr[batch])
        dec = decode.PageGaugeSegmentedDecode(ws)
        dec.plan(w.old_indptr[:batch + 1], w.old_indices[:n_old], w.old_last_page_len[:batch],
                 w.tail_indptr[:batch + 1], w.tail_indices[:n_tail], w.tail_last_page_len[:batch],
                 fixed_split_size=split, tail_split_size=16)
        assert dec._state.plan.max_items_per_request == max(items, 4 if batch > 1 else 0)
        out, lse = dec.run(w.query[:batch], (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                           (w.tail_k, w.tail_v), w.value_center[:batch], return_lse=True)
        torch.cuda.synchronize()
        results.append((out[0].clone(), lse[0].clone()))
    (out_blocks, lse_blocks), (out_rows, lse_rows) = results
    assert torch.equal(out_rows, out_blocks) and torch.equal(lse_rows, lse_blocks)
    ref_out, ref_lse, ref64 = oracle_decode(w)
    assert fp16_parity(out_rows, ref_out[0], ref64[0])["ok"]
    assert max_abs(lse_rows, ref_lse[0]) <= 2e-3
