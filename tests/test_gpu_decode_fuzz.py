"""Seeded random decode problems against the float64 oracle: ragged batches
of 1-6 requests, INT8 histories of 1-256 pages, FP16 tails of 1-16 pages
with a random fill of their last page, a permuted shared page pool, and
the planner's own split or a fixed one.  Tolerance as everywhere: out and
lse max-abs <= 2e-3."""

from __future__ import annotations

import random

import pytest
import torch

from tests.helpers import max_abs, oracle_decode

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
    ref_out, ref_lse, _ = oracle_decode(w)
    err, lerr = max_abs(out, ref_out), max_abs(lse, ref_lse)
    print(f"fuzz {index}: lengths {lengths} tail {tail_pages} split {split} last {last} "
          f"items {dec.num_work_items}: out {err:.2e} lse {lerr:.2e}", flush=True)
    assert err <= 2e-3 and lerr <= 2e-3
