"""Size-independent properties of the paged decode at BASELINE's full sizes.

* Physical layout does not matter: moving every page of the B1/49K cache to
  another physical slot (codes, scales and FP16 tail pages alike) and
  rewriting the page tables to match leaves out and lse bit-identical, since
  each work item sees the same logical data in the same order.  This pins the
  page-id lookup (patches/flashinfer-0.6.17-page-gauge-int8.patch:157-175)
  at 3056 + 16 pages.
* Page-id collisions: several logical pages naming one physical page (the
  reference clamps ids but never forbids repeats) read that page's data each
  time, checked against the float64 oracle.
* Batch independence: a request decoded inside the B8 ragged batch gives the
  same bits as the same request decoded alone with the same per-request
  items.
"""

from __future__ import annotations

import pytest
import torch

from tests.helpers import max_abs, oracle_decode

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def workspace(cuda):
    return torch.empty(64 << 20, dtype=torch.uint8, device=cuda)


def _run(w, workspace, split=None):
    from pagegauge_amd import decode

    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, fixed_split_size=split)
    out, lse = dec.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                       w.value_center, return_lse=True)
    torch.cuda.synchronize()
    return out.clone(), lse.clone()


def _relocate(pool, indices, perm):
    """Move physical page p of ``pool`` to slot perm[p]; returns the new pool
    and the page table that names the same logical pages."""
    moved = torch.empty_like(pool)
    moved[perm.long()] = pool
    return moved, perm[indices.long()].to(torch.int32).contiguous()


def test_b1_49k_physical_layout_is_invisible(cuda, workspace):
    from pagegauge_amd import workloads

    w = workloads.b1_49k(20260840, device=cuda)
    out, lse = _run(w, workspace)
    gen = torch.Generator().manual_seed(5)
    perm = torch.randperm(w.k_codes.shape[0], generator=gen).to(torch.int32).to(cuda)
    w.k_codes, old = _relocate(w.k_codes, w.old_indices, perm)
    w.v_codes, _ = _relocate(w.v_codes, w.old_indices, perm)
    w.k_scale, _ = _relocate(w.k_scale, w.old_indices, perm)
    w.v_scale, _ = _relocate(w.v_scale, w.old_indices, perm)
    w.old_indices = old
    tperm = torch.randperm(w.tail_k.shape[0], generator=gen).to(torch.int32).to(cuda)
    w.tail_k, tail = _relocate(w.tail_k, w.tail_indices, tperm)
    w.tail_v, _ = _relocate(w.tail_v, w.tail_indices, tperm)
    w.tail_indices = tail
    out2, lse2 = _run(w, workspace)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)


@pytest.mark.parametrize("split", [None, 3])
def test_repeated_page_ids_read_the_same_page(cuda, workspace, split):
    from pagegauge_amd import workloads

    w = workloads.build_decode_workload([2048 + 256, 1024 + 256], 20260841, device=cuda)
    ids = w.old_indices.clone()
    ids[1::3] = ids[0]                      # every third logical page names page ids[0]
    ids[-1] = ids[2]
    w.old_indices = ids.contiguous()
    tail = w.tail_indices.clone()
    tail[0] = tail[-1]                      # a tail ring slot named twice
    w.tail_indices = tail.contiguous()
    out, lse = _run(w, workspace, split)
    ref_out, ref_lse, _ = oracle_decode(w)
    assert max_abs(out, ref_out) <= 2e-3 and max_abs(lse, ref_lse) <= 2e-3


def test_a_request_decodes_alike_alone_and_in_the_ragged_batch(cuda, workspace):
    from pagegauge_amd import workloads

    w = workloads.b8_ragged(20260840, device=cuda)
    out, lse = _run(w, workspace, split=16)
    r = 3
    ob, oe = int(w.old_indptr[r]), int(w.old_indptr[r + 1])
    tb, te = int(w.tail_indptr[r]), int(w.tail_indptr[r + 1])
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=cuda)  # noqa: E731
    w.query = w.query[r:r + 1].contiguous()
    w.old_indices = w.old_indices[ob:oe].contiguous()
    w.old_indptr = i32([0, oe - ob])
    w.old_last_page_len = w.old_last_page_len[r:r + 1].contiguous()
    w.tail_indices = w.tail_indices[tb:te].contiguous()
    w.tail_indptr = i32([0, te - tb])
    w.tail_last_page_len = w.tail_last_page_len[r:r + 1].contiguous()
    w.value_center = w.value_center[r:r + 1].contiguous()
    alone, alone_lse = _run(w, workspace, split=16)
    assert torch.equal(alone[0], out[r]) and torch.equal(alone_lse[0], lse[r])
