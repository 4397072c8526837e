"""A served decode batch on the GPU: ragged requests over a shared, shuffled
physical page pool and per-lease exact sidecars (prefix / static suffix /
tail ring), driven by the serving metadata (``pagegauge_amd.serving``).

Every step runs K2 through the serving tables (``rope_append_page_gauge_slots``)
and K1 over the step's history / exact tables, and is checked against the
oracle on a numpy mirror of the caches: the cache updates bit-exact, the
attention within 2e-3.  Midway a request retires and a new one is admitted
into its sidecar slot and pages (lease generation 2)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import assert_bit_equal, cpu, max_abs

pytestmark = pytest.mark.gpu

HQ, HKV, D, PAGE = 32, 8, 128, 16


class Pool:
    """Physical pages handed out in a fixed shuffled order; freed pages return."""

    def __init__(self, n, gen):
        self.free = torch.randperm(n, generator=gen).tolist()

    def take(self, count):
        pages, self.free = self.free[:count], self.free[count:]
        return pages

    def give(self, pages):
        self.free = list(pages) + self.free             # reused first: stale pages get rewritten


def _prefill(d, lease, prompt, table, gen, pol, cuda):
    """Populate one request: exact centers, INT8 codes of its whole pages in
    their physical pages, centered FP16 exact pages (and the partial page)."""
    from pagegauge_amd import serving as sv
    from pagegauge_amd.update import prefill_page_gauge, token_major_centers

    k = (torch.randn(prompt, HKV, D, generator=gen)).to(torch.float16).to(cuda)
    v = (torch.randn(prompt, HKV, D, generator=gen)).to(torch.float16).to(cuda)
    kc, vc = token_major_centers(k, v, d["key_center"][lease.slot], d["value_center"][lease.slot])
    whole = prompt // PAGE
    part = sv.partition(prompt, prompt, pol)
    exact_map = torch.full((whole,), -1, dtype=torch.int32)
    for p in part["exact"]:
        if p < whole:
            exact_map[p] = sv.exact_slot(p, prompt, lease.slot, pol)
    tmp = [torch.empty(whole, PAGE, HKV, D, device=cuda, dtype=torch.int8) for _ in range(2)]
    sc = [torch.empty(whole, HKV, device=cuda, dtype=torch.float16) for _ in range(2)]
    prefill_page_gauge(k[:whole * PAGE], v[:whole * PAGE], kc, vc, tmp[0], tmp[1], sc[0], sc[1],
                       exact_map.to(cuda), d["exact_k"], d["exact_v"])
    ids = torch.tensor(table[:whole], device=cuda, dtype=torch.long)
    d["codes_k"].index_copy_(0, ids, tmp[0])
    d["codes_v"].index_copy_(0, ids, tmp[1])
    d["scales_k"].index_copy_(0, ids, sc[0])
    d["scales_v"].index_copy_(0, ids, sc[1])
    if prompt % PAGE:                                  # the partial page lives in the tail ring
        slot = sv.exact_slot(whole, prompt, lease.slot, pol)
        rows = prompt - whole * PAGE
        d["exact_k"][slot, :rows] = (k[whole * PAGE:].float() - kc.float()).half()
        d["exact_v"][slot, :rows] = (v[whole * PAGE:].float() - vc.float()).half()


def test_served_batch_matches_the_oracle_step_by_step(cuda):
    from pagegauge_amd import decode, serving as sv
    from pagegauge_amd.decoder import rope_tables
    from pagegauge_amd.runtime import load_append_extension

    ext = load_append_extension()
    gen = torch.Generator().manual_seed(20260860)
    pol = sv.Policy(prefix_pages=2, suffix_pages=4, tail_pages=3)
    ledger = sv.Ledger(3, pol)
    n_pages = 320
    pool = Pool(n_pages, gen)
    d = {"codes_k": torch.zeros(n_pages, PAGE, HKV, D, device=cuda, dtype=torch.int8),
         "scales_k": torch.zeros(n_pages, HKV, device=cuda, dtype=torch.float16),
         "exact_k": torch.zeros(3 * pol.storage_pages, PAGE, HKV, D, device=cuda, dtype=torch.float16),
         "key_center": torch.zeros(3, HKV, D, device=cuda, dtype=torch.float16)}
    d["codes_v"], d["scales_v"] = torch.zeros_like(d["codes_k"]), torch.zeros_like(d["scales_k"])
    d["exact_v"], d["value_center"] = torch.zeros_like(d["exact_k"]), torch.zeros_like(d["key_center"])
    cos, sin = (t.to(cuda) for t in rope_tables(4096, 1.0e6))
    tables = {}

    def admit(name, prompt):
        table = pool.take((prompt + PAGE - 1) // PAGE)
        lease = ledger.admit(name, prompt, table, ready=True)
        tables[name] = table
        _prefill(d, lease, prompt, table, gen, pol, cuda)
        return lease

    leases = {n: admit(n, p) for n, p in (("a", 800), ("b", 1000), ("c", 1208))}
    torch.cuda.synchronize()
    mirror = {k: cpu(v).copy() for k, v in d.items()}
    workspace = torch.empty(16 << 20, dtype=torch.uint8, device=cuda)
    cache_keys = ("exact_k", "exact_v", "codes_k", "codes_v", "scales_k", "scales_v")
    worst, finalized, read_back = 0.0, set(), set()
    for step in range(64):
        if step == 24:                                         # retire a, admit d into its slot
            for key in cache_keys:
                assert_bit_equal(d[key], mirror[key], f"{key} before the retirement")
            retired = tables.pop("a")
            ledger.release(leases.pop("a"))
            pool.give(retired)
            leases["d"] = admit("d", 904)
            assert leases["d"].slot == 0 and leases["d"].generation == 2
            assert set(retired) <= set(tables["d"])            # d reuses all of a's pages
            torch.cuda.synchronize()
            for k in cache_keys + ("key_center", "value_center"):
                mirror[k] = cpu(d[k]).copy()
        scheduled = []
        for name, lease in leases.items():
            position = ledger.view(lease).current_tokens
            if position % PAGE == 0:
                tables[name] = tables[name] + pool.take(1)
            scheduled.append((lease, position, tables[name]))
        batch = ledger.stage_decode(scheduled)
        t = sv.decode_tables(batch, pol, device=cuda)
        read_back |= finalized & set(cpu(t.old_indices).tolist())
        finalized |= {table[position // PAGE] for _, position, table in scheduled
                      if position % PAGE == PAGE - 1}
        b = len(scheduled)
        q = torch.randn(b, HQ, D, generator=gen).to(torch.float16)
        k = torch.randn(b, HKV, D, generator=gen).to(torch.float16)
        v = torch.randn(b, HKV, D, generator=gen).to(torch.float16)
        slot_ids = t.request_slots.long()
        kc, vc = d["key_center"][slot_ids].contiguous(), d["value_center"][slot_ids].contiguous()
        rq = torch.empty(b, HQ, D, device=cuda, dtype=torch.float16)
        ext.rope_append_page_gauge_slots(q.to(cuda), k.to(cuda), v.to(cuda), cos, sin, t.positions,
                                         t.exact_page_ids, t.code_page_ids, kc, vc, rq, d["exact_k"],
                                         d["exact_v"], d["codes_k"], d["codes_v"], d["scales_k"],
                                         d["scales_v"])
        m_rq = np.zeros((b, HQ, D), np.float16)
        oracle.rope_append_page_gauge_slots(
            q.numpy(), k.numpy(), v.numpy(), cpu(cos), cpu(sin), cpu(t.positions),
            cpu(t.exact_page_ids), cpu(t.code_page_ids), cpu(kc), cpu(vc), m_rq, mirror["exact_k"],
            mirror["exact_v"], mirror["codes_k"], mirror["codes_v"], mirror["scales_k"],
            mirror["scales_v"])
        dec = decode.PageGaugeSegmentedDecode(workspace)
        dec.plan(t.old_indptr, t.old_indices, t.old_last_page_len, t.exact_indptr, t.exact_indices,
                 t.exact_last_page_len)
        out, lse = dec.run(rq, (d["codes_k"], d["codes_v"]), d["scales_k"], d["scales_v"],
                           (d["exact_k"], d["exact_v"]), value_center=vc, return_lse=True)
        want, want_lse, _ = oracle.decode(
            m_rq, mirror["codes_k"], mirror["codes_v"], cpu(t.old_indptr), cpu(t.old_indices),
            cpu(t.old_last_page_len), D ** -0.5, k_scale=mirror["scales_k"],
            v_scale=mirror["scales_v"], tail_k=mirror["exact_k"], tail_v=mirror["exact_v"],
            tail_indptr=cpu(t.exact_indptr), tail_indices=cpu(t.exact_indices),
            tail_last_page_len=cpu(t.exact_last_page_len), value_center=cpu(vc))
        torch.cuda.synchronize()
        assert_bit_equal(rq, m_rq, f"rotated query, step {step}")
        worst = max(worst, max_abs(out, want))
        assert max_abs(out, want) <= 2e-3, step
        assert max_abs(lse, want_lse) <= 2e-3, step
        ledger.commit_decode(batch)
    print(f"served decode: 64 steps, max |out - oracle| = {worst:.3g}, "
          f"{len(read_back)} decode-finalized pages read back as INT8 history")
    for key in cache_keys:
        assert_bit_equal(d[key], mirror[key], key)
    # pages completed by K2 during decode left the tail ring and were read by
    # K1 from their physical INT8 pages
    assert len(read_back) >= 2


def test_slots_variant_equals_positions_variant_on_request_major_tables(cuda):
    """With request-major ids the serving kernel is the per-request-position
    kernel (same rows, same codes)."""
    from pagegauge_amd.decoder import rope_tables
    from pagegauge_amd.runtime import load_append_extension

    ext = load_append_extension()
    gen = torch.Generator().manual_seed(5)
    batch, ring, code_pages = 3, 4, 6
    cos, sin = (x.to(cuda) for x in rope_tables(96, 1.0e6))
    kc = (torch.randn(batch, HKV, D, generator=gen) * 0.1).half().to(cuda)
    vc = (torch.randn(batch, HKV, D, generator=gen) * 0.1).half().to(cuda)
    bufs = []
    for _ in range(2):
        bufs.append(dict(
            rq=torch.zeros(batch, HQ, D, device=cuda, dtype=torch.float16),
            ek=torch.zeros(batch * ring, PAGE, HKV, D, device=cuda, dtype=torch.float16),
            ev=torch.zeros(batch * ring, PAGE, HKV, D, device=cuda, dtype=torch.float16),
            ck=torch.zeros(batch * code_pages, PAGE, HKV, D, device=cuda, dtype=torch.int8),
            cv=torch.zeros(batch * code_pages, PAGE, HKV, D, device=cuda, dtype=torch.int8),
            sk=torch.zeros(batch * code_pages, HKV, device=cuda, dtype=torch.float16),
            sv=torch.zeros(batch * code_pages, HKV, device=cuda, dtype=torch.float16)))
    start = torch.tensor([3, 17, 40])
    for step in range(40):
        pos = start + step
        q = torch.randn(batch, HQ, D, generator=gen).half().to(cuda)
        k = torch.randn(batch, HKV, D, generator=gen).half().to(cuda)
        v = torch.randn(batch, HKV, D, generator=gen).half().to(cuda)
        p = pos.to(torch.int32).to(cuda)
        page = pos // PAGE
        exact_ids = (torch.arange(batch) * ring + page % ring).to(torch.int32).to(cuda)
        code_ids = (torch.arange(batch) * code_pages + page).to(torch.int32).to(cuda)
        a, s = bufs
        ext.rope_append_page_gauge_positions(q, k, v, cos, sin, p, kc, vc, a["rq"], a["ek"], a["ev"],
                                             a["ck"], a["cv"], a["sk"], a["sv"], 0)
        ext.rope_append_page_gauge_slots(q, k, v, cos, sin, p, exact_ids, code_ids, kc, vc, s["rq"],
                                         s["ek"], s["ev"], s["ck"], s["cv"], s["sk"], s["sv"])
    torch.cuda.synchronize()
    for key in bufs[0]:
        assert torch.equal(bufs[0][key], bufs[1][key]), key
