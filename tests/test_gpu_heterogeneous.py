"""GPU parity of the heterogeneous one-table decode (``pg_decode_run_heterogeneous``)
against the oracle, on the reference's nine boundary cases
(diagnostics/benchmark_heterogeneous_fa2_correctness.py:63-73).

As in the reference fixture, exact pages that no table entry references are
NaN, and so are the rows of the last page past its last token, so a kernel
that lets them reach the output fails.  Fixed split sizes of 1-3 pages
make work items straddle the INT8/FP16 boundary; moving the boundary in place
(table entry + old_kv_len) must not need a new plan."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import fp16_parity, max_abs

pytestmark = pytest.mark.gpu

CASES = [("old_only", 256, 256, 1), ("exact_only_last1", 0, 1, 2), ("exact_only_last15", 0, 15, 2),
         ("exact_only_last16", 0, 16, 2), ("boundary_last1", 16, 17, 4),
         ("boundary_last15", 16, 31, 4), ("boundary_last16", 16, 32, 4),
         ("boundary_after_full_cta", 144, 176, 4), ("ring_wrap_last15", 144, 191, 4)]


def _fixture(old_tokens, total_tokens, ring_pages, batch, seed):
    rng = np.random.default_rng(seed)
    hkv = 8
    total_pages = -(-total_tokens // 16)
    old_pages = old_tokens // 16
    store = max(old_pages, 1)
    centered_k = (rng.standard_normal((batch, total_pages, 16, hkv, 128)) * 0.08).astype(np.float16)
    centered_v = (rng.standard_normal((batch, total_pages, 16, hkv, 128)) * 0.08).astype(np.float16)
    k_codes = np.full((batch * store, 16, hkv, 128), -91, np.int8)
    v_codes = np.full_like(k_codes, 73)
    k_scale = np.full((batch * store, hkv), 0.0031, np.float16)
    v_scale = np.full((batch * store, hkv), 0.0047, np.float16)
    exact_k = np.full((batch * ring_pages, 16, hkv, 128), np.nan, np.float16)
    exact_v = np.full_like(exact_k, np.nan)
    indices = []
    for r in range(batch):
        if old_pages:
            ck, _, sk, _, _ = oracle.quantize_page_gauge(centered_k[r, :old_pages],
                                                         center=np.zeros((hkv, 128), np.float16))
            cv, _, sv, _, _ = oracle.quantize_page_gauge(centered_v[r, :old_pages],
                                                         center=np.zeros((hkv, 128), np.float16))
            k_codes[r * store:r * store + old_pages] = ck
            v_codes[r * store:r * store + old_pages] = cv
            k_scale[r * store:r * store + old_pages] = sk
            v_scale[r * store:r * store + old_pages] = sv
        for page in range(total_pages):
            if page < old_pages:
                indices.append(r * store + page)
            else:
                slot = r * ring_pages + page % ring_pages
                exact_k[slot] = centered_k[r, page]
                exact_v[slot] = centered_v[r, page]
                if page == total_pages - 1:           # rows past the last token: NaN too
                    last = (total_tokens - 1) % 16 + 1
                    exact_k[slot, last:] = np.nan
                    exact_v[slot, last:] = np.nan
                indices.append(slot)
    query = (rng.standard_normal((batch, 32, 128)) * 0.35).astype(np.float16)
    center = (rng.standard_normal((batch, hkv, 128)) * 0.025).astype(np.float16)
    if old_tokens == 0:
        center[:] = 0
    return dict(query=query, k_codes=k_codes, v_codes=v_codes, k_scale=k_scale, v_scale=v_scale,
                exact_k=exact_k, exact_v=exact_v,
                indptr=np.arange(batch + 1, dtype=np.int32) * total_pages,
                indices=np.array(indices, dtype=np.int32),
                last=np.full(batch, (total_tokens - 1) % 16 + 1, np.int32),
                old_len=np.full(batch, old_tokens, np.int32), center=center)


def _oracle(f):
    return oracle.decode_heterogeneous(f["query"], f["k_codes"], f["v_codes"], f["k_scale"],
                                       f["v_scale"], f["exact_k"], f["exact_v"], f["indptr"],
                                       f["indices"], f["last"], f["old_len"], 128 ** -0.5,
                                       value_center=f["center"])


def _device(f, cuda):
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(cuda) for k, v in f.items()}


def _run(d, split, cuda, hint=0):
    from pagegauge_amd import decode

    ws = torch.empty(8 << 20, dtype=torch.uint8, device=cuda)
    wrapper = decode.make_heterogeneous_page_gauge_wrapper(None, ws)
    wrapper.plan(d["indptr"], d["indices"], d["last"], 32, 8, 128, 16, fixed_split_size=split or None,
                 exact_tail_pages_hint=hint)
    decode.validate_heterogeneous_run_inputs(d["query"], d["k_codes"], d["v_codes"], d["k_scale"],
                                             d["v_scale"], d["exact_k"], d["exact_v"], d["old_len"],
                                             d["center"])
    out, lse = wrapper.run(d["query"], (d["k_codes"], d["v_codes"]), d["k_scale"], d["v_scale"],
                           d["exact_k"], d["exact_v"], d["old_len"], d["center"], 128 ** -0.5,
                           return_lse=True)
    torch.cuda.synchronize()
    return wrapper, out, lse


@pytest.mark.parametrize("split", [0, 1, 2, 3])
@pytest.mark.parametrize("name,old_tokens,total_tokens,ring_pages", CASES)
def test_heterogeneous_matches_oracle(cuda, name, old_tokens, total_tokens, ring_pages, split):
    print(f"heterogeneous {name} split={split}", flush=True)
    f = _fixture(old_tokens, total_tokens, ring_pages, batch=3, seed=sum(map(ord, name)) + split)
    want16, want_lse, want64 = _oracle(f)
    _, out, lse = _run(_device(f, cuda), split, cuda)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    assert fp16_parity(out, want16, want64)["ok"], name
    assert max_abs(lse, want_lse) <= 2e-3, name


@pytest.mark.parametrize("hint", [1, 4, 40])
@pytest.mark.parametrize("name,old_tokens,total_tokens,ring_pages", CASES)
def test_exact_tail_hint_changes_balance_not_results(cuda, name, old_tokens, total_tokens,
                                                      ring_pages, hint):
    """The planning hint may match the real INT8/FP16 boundary or not (1 and
    40 trailing pages against rings of 1-4 pages); results stay the oracle's."""
    print(f"heterogeneous hint {name} hint={hint}", flush=True)
    f = _fixture(old_tokens, total_tokens, ring_pages, batch=3, seed=sum(map(ord, name)) + hint)
    want16, want_lse, want64 = _oracle(f)
    _, out, lse = _run(_device(f, cuda), 0, cuda, hint=hint)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    assert fp16_parity(out, want16, want64)["ok"], name
    assert max_abs(lse, want_lse) <= 2e-3, name


def test_moving_the_boundary_needs_no_new_plan(cuda):
    # ring_wrap_last15 with 9 INT8 pages, then page 8 moves to the exact pool
    f = _fixture(144, 191, 4, batch=1, seed=7)
    d = _device(f, cuda)
    wrapper, out, _ = _run(d, 2, cuda)
    want16, _, want64 = _oracle(f)
    assert fp16_parity(out, want16, want64)["ok"]
    # move logical page 8 into a free exact slot (the ring has 4 slots: pages 9..11 use 1..3)
    slot = 0
    codes_k = f["k_codes"][8].astype(np.float64) * f["k_scale"][8].astype(np.float64)[None, :, None]
    codes_v = f["v_codes"][8].astype(np.float64) * f["v_scale"][8].astype(np.float64)[None, :, None]
    f["exact_k"][slot] = codes_k.astype(np.float16)
    f["exact_v"][slot] = codes_v.astype(np.float16)
    f["indices"][8] = slot
    f["old_len"][0] = 128
    d["exact_k"].copy_(torch.from_numpy(f["exact_k"]))
    d["exact_v"].copy_(torch.from_numpy(f["exact_v"]))
    d["indices"].copy_(torch.from_numpy(f["indices"]))
    d["old_len"].fill_(128)
    out2 = wrapper.run(d["query"], (d["k_codes"], d["v_codes"]), d["k_scale"], d["v_scale"],
                       d["exact_k"], d["exact_v"], d["old_len"], d["center"])
    torch.cuda.synchronize()
    want16, _, want64 = _oracle(f)
    assert fp16_parity(out2, want16, want64)["ok"]
    assert max_abs(out2, out) <= 2e-3          # same logical cache, other representation


def test_heterogeneous_equals_segmented_run(cuda):
    """The unified table and the two-segment plan over the same pages agree."""
    from pagegauge_amd import decode

    f = _fixture(144 * 8, 144 * 8 + 100, 8, batch=2, seed=11)
    d = _device(f, cuda)
    _, out_h, lse_h = _run(d, 0, cuda)
    total_pages = int(f["indptr"][1])
    old_pages = int(f["old_len"][0]) // 16
    old_idx = np.concatenate([f["indices"][r * total_pages:r * total_pages + old_pages] for r in range(2)])
    tail_idx = np.concatenate([f["indices"][r * total_pages + old_pages:(r + 1) * total_pages]
                               for r in range(2)])
    seg = decode.PageGaugeSegmentedDecode(torch.empty(8 << 20, dtype=torch.uint8, device=cuda))
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(cuda)  # noqa: E731
    seg.plan(t([0, old_pages, 2 * old_pages]), t(old_idx), t([16, 16]),
             t([0, total_pages - old_pages, 2 * (total_pages - old_pages)]), t(tail_idx), d["last"])
    out_s, lse_s = seg.run(d["query"], (d["k_codes"], d["v_codes"]), d["k_scale"], d["v_scale"],
                           (d["exact_k"], d["exact_v"]), value_center=d["center"], return_lse=True)
    torch.cuda.synchronize()
    assert max_abs(out_h, out_s) <= 1e-3 and max_abs(lse_h, lse_s) <= 1e-4


def test_heterogeneous_run_validation(cuda):
    from pagegauge_amd import decode

    f = _fixture(16, 31, 4, batch=1, seed=3)
    d = _device(f, cuda)
    with pytest.raises(ValueError, match="page-aligned"):
        decode.validate_heterogeneous_run_inputs(d["query"], d["k_codes"], d["v_codes"],
                                                 d["k_scale"], d["v_scale"], d["exact_k"],
                                                 d["exact_v"], d["old_len"] + 1, d["center"])
    with pytest.raises(ValueError, match="old_k_cache must be contiguous CUDA"):
        decode.validate_heterogeneous_run_inputs(d["query"], d["k_codes"].half(), d["v_codes"],
                                                 d["k_scale"], d["v_scale"], d["exact_k"],
                                                 d["exact_v"], d["old_len"], d["center"])
    wrapper = decode.make_heterogeneous_page_gauge_wrapper(
        None, torch.empty(1 << 20, dtype=torch.uint8, device=cuda))
    with pytest.raises(RuntimeError, match="plan"):
        wrapper.run(d["query"], (d["k_codes"], d["v_codes"]), d["k_scale"], d["v_scale"],
                    d["exact_k"], d["exact_v"], d["old_len"], d["center"])


@pytest.mark.parametrize("lengths", [[49152], [20480] * 4])
def test_hinted_heterogeneous_is_bit_identical_to_segmented(cuda, lengths):
    """With the exact-tail hint of the ring's 16 pages the unified-table plan
    cuts the same items as the segmented plan (config 2's B1/49K and the
    paper's B4 x 20K shape), so the two calls return the same bits: the
    heterogeneous items take their INT8 pages and page ids exactly as the
    segmented INT8 items do."""
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload(lengths, 20260840, device=cuda)
    seg = decode.PageGaugeSegmentedDecode(torch.empty(64 << 20, dtype=torch.uint8, device=cuda))
    seg.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len)
    out_s, lse_s = seg.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                           (w.tail_k, w.tail_v), w.value_center, return_lse=True)
    old_ptr, tail_ptr = w.old_indptr.tolist(), w.tail_indptr.tolist()
    old_idx, tail_idx = w.old_indices.cpu(), w.tail_indices.cpu()
    rows, indptr, old_len = [], [0], []
    for b in range(w.batch):
        rows += [old_idx[old_ptr[b]:old_ptr[b + 1]], tail_idx[tail_ptr[b]:tail_ptr[b + 1]]]
        indptr.append(indptr[-1] + old_ptr[b + 1] - old_ptr[b] + tail_ptr[b + 1] - tail_ptr[b])
        old_len.append(16 * (old_ptr[b + 1] - old_ptr[b]))
    unified = torch.cat(rows).to(cuda)
    het = decode.make_heterogeneous_page_gauge_wrapper(
        None, torch.empty(64 << 20, dtype=torch.uint8, device=cuda))
    het.plan(torch.tensor(indptr, dtype=torch.int32), unified, w.tail_last_page_len, 32, 8, 128, 16,
             exact_tail_pages_hint=16)
    out_h, lse_h = het.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, w.tail_k,
                           w.tail_v, torch.tensor(old_len, dtype=torch.int32, device=cuda),
                           w.value_center, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out_h, out_s) and torch.equal(lse_h, lse_s)
