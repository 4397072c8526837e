"""Seeded random decode problems against the float64 oracle: ragged batches
of 1-6 requests, INT8 histories of 1-256 pages, FP16 tails of 1-16 pages
with a random fill of their last page, a permuted shared page pool, and
the planner's own split or a fixed one; the segmented decode and the
heterogeneous one-table decode of the same pages.  Tolerance: lse max-abs
<= 2e-3, out within 2e-3 of the FP16-rounded oracle or a one-ulp rounding
flip of a value on a rounding boundary (``helpers.fp16_parity``)."""

from __future__ import annotations

import random

import pytest
import torch

from tests.helpers import fp16_parity, max_abs, oracle_decode

pytestmark = pytest.mark.gpu

CASES = 16


def _case(index):
    rng = random.Random(20260900 + index)
    batch = rng.randint(1, 6)
    tail_pages = rng.choice([1, 4, 16])
    lengths = [16 * (tail_pages + rng.randint(1, 256)) for _ in range(batch)]
    split = rng.choice([None, None, 1, 2, 5, 16, 64])
    last = [rng.randint(1, 16) for _ in range(batch)]
    return lengths, tail_pages, split, last


@pytest.fixture(scope="module")
def workspace(cuda):
    return torch.empty(64 << 20, dtype=torch.uint8, device=cuda)


@pytest.mark.parametrize("index", range(CASES))
def test_random_decode_matches_oracle(cuda, workspace, index):
    from pagegauge_amd import decode, workloads

    lengths, tail_pages, split, last = _case(index)
    w = workloads.build_decode_workload(lengths, 20260900 + index, device=cuda,
                                        tail_tokens=16 * tail_pages)
    w.tail_last_page_len = torch.tensor(last, dtype=torch.int32, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, fixed_split_size=split)
    out, lse = dec.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                       w.value_center, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref64 = oracle_decode(w)
    par, lerr = fp16_parity(out, ref_out, ref64), max_abs(lse, ref_lse)
    print(f"fuzz {index}: lengths {lengths} tail {tail_pages} split {split} last {last} "
          f"items {dec.num_work_items}: {par} lse {lerr:.2e}", flush=True)
    assert par["ok"] and lerr <= 2e-3


def _unified(w, device):
    """One table per request: its INT8 pages, then its FP16 ring pages."""
    old_ptr, tail_ptr = w.old_indptr.tolist(), w.tail_indptr.tolist()
    old_idx, tail_idx = w.old_indices.cpu(), w.tail_indices.cpu()
    rows, indptr, old_len = [], [0], []
    for b in range(w.batch):
        rows += [old_idx[old_ptr[b]:old_ptr[b + 1]], tail_idx[tail_ptr[b]:tail_ptr[b + 1]]]
        indptr.append(indptr[-1] + old_ptr[b + 1] - old_ptr[b] + tail_ptr[b + 1] - tail_ptr[b])
        old_len.append(16 * (old_ptr[b + 1] - old_ptr[b]))
    return (torch.tensor(indptr, dtype=torch.int32), torch.cat(rows).to(device),
            torch.tensor(old_len, dtype=torch.int32, device=device))


# seed 75 of this generator puts an output of -7.6894518 (float64) 1.3e-6
# from the FP16 rounding midpoint -7.6894531: the kernel, 1.6e-7 from the
# float64 value, rounds to the other neighbour (one ulp = 3.9e-3 away)
@pytest.mark.parametrize("index", list(range(8)) + [75])
def test_random_heterogeneous_decode_matches_oracle(cuda, workspace, index):
    from pagegauge_amd import decode, workloads

    rng = random.Random(20261900 + index)
    batch = rng.randint(1, 6)
    tail_pages = rng.choice([1, 4, 16])
    lengths = [16 * (tail_pages + rng.randint(1, 256)) for _ in range(batch)]
    split = rng.choice([None, None, 1, 2, 5, 16, 64])
    hint = rng.choice([0, tail_pages])
    last = [rng.randint(1, 16) for _ in range(batch)]
    w = workloads.build_decode_workload(lengths, 20261900 + index, device=cuda,
                                        tail_tokens=16 * tail_pages)
    w.tail_last_page_len = torch.tensor(last, dtype=torch.int32, device=cuda)
    indptr, unified, old_kv_len = _unified(w, cuda)
    het = decode.make_heterogeneous_page_gauge_wrapper(None, workspace)
    het.plan(indptr, unified, w.tail_last_page_len, 32, 8, 128, 16, fixed_split_size=split,
             exact_tail_pages_hint=hint)
    out = het.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, w.tail_k, w.tail_v,
                  old_kv_len, w.value_center)
    torch.cuda.synchronize()
    ref_out, _, ref64 = oracle_decode(w)
    par = fp16_parity(out, ref_out, ref64)
    print(f"heterogeneous {index}: lengths {lengths} tail {tail_pages} split {split} hint {hint} "
          f"last {last}: {par}", flush=True)
    assert par["ok"]
    if index == 75:
        assert par["boundary_flips"] >= 1 and par["max_interval_gap"] < 1e-5
