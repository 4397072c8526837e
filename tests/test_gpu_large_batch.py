"""Serving-sized decode batches: 64, 256 and 1024 requests of ragged
lengths (1-256 INT8 pages each behind a 16-page FP16 ring with a random
fill of its last page) in one shuffled pool, through the segmented decode
and the heterogeneous one-table decode, against the float64 oracle (out:
``helpers.fp16_parity``; lse max-abs <= 2e-3)."""

from __future__ import annotations

import random

import pytest
import torch

from tests.helpers import fp16_parity, max_abs, oracle_decode

pytestmark = pytest.mark.gpu


def _workload(batch, max_pages, seed, cuda):
    from pagegauge_amd import workloads

    rng = random.Random(seed)
    lengths = [16 * (16 + rng.randint(1, max_pages)) for _ in range(batch)]
    w = workloads.build_decode_workload(lengths, seed, device=cuda, tail_tokens=256)
    w.tail_last_page_len = torch.tensor([rng.randint(1, 16) for _ in range(batch)],
                                        dtype=torch.int32, device=cuda)
    return w


@pytest.mark.parametrize("batch,max_pages,split", [(64, 256, None), (256, 64, None),
                                                    (256, 64, 8), (1024, 8, None)])
def test_large_batch_segmented_decode(cuda, batch, max_pages, split):
    from pagegauge_amd import decode

    seed = 20261210 + batch + (split or 0)
    print(f"large batch B={batch} max_pages={max_pages} split={split}", flush=True)
    w = _workload(batch, max_pages, seed, cuda)
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(ws)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, fixed_split_size=split)
    out, lse = dec.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                       w.value_center, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref64 = oracle_decode(w)
    par, lerr = fp16_parity(out, ref_out, ref64), max_abs(lse, ref_lse)
    plan = dec._state.plan
    print(f"  items {plan.num_items} waves/wg {plan.waves_per_block}: {par} lse {lerr:.2e}",
          flush=True)
    assert par["ok"] and lerr <= 2e-3


def test_large_batch_heterogeneous_decode(cuda):
    from pagegauge_amd import decode

    print("large batch heterogeneous B=256", flush=True)
    w = _workload(256, 64, 20261299, cuda)
    old_ptr, tail_ptr = w.old_indptr.tolist(), w.tail_indptr.tolist()
    old_idx, tail_idx = w.old_indices.cpu(), w.tail_indices.cpu()
    rows, indptr, old_len = [], [0], []
    for b in range(w.batch):
        rows += [old_idx[old_ptr[b]:old_ptr[b + 1]], tail_idx[tail_ptr[b]:tail_ptr[b + 1]]]
        indptr.append(indptr[-1] + old_ptr[b + 1] - old_ptr[b] + tail_ptr[b + 1] - tail_ptr[b])
        old_len.append(16 * (old_ptr[b + 1] - old_ptr[b]))
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=cuda)
    het = decode.make_heterogeneous_page_gauge_wrapper(None, ws)
    het.plan(torch.tensor(indptr, dtype=torch.int32), torch.cat(rows).to(cuda),
             w.tail_last_page_len, 32, 8, 128, 16, exact_tail_pages_hint=16)
    out = het.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, w.tail_k, w.tail_v,
                  torch.tensor(old_len, dtype=torch.int32, device=cuda), w.value_center)
    torch.cuda.synchronize()
    ref_out, _, ref64 = oracle_decode(w)
    par = fp16_parity(out, ref_out, ref64)
    print(f"  {par}", flush=True)
    assert par["ok"]
