"""Page pools past 4 GiB: every kernel that takes page ids (K1 segmented and
heterogeneous decode, the fused exact tail, K2 through serving slots and
the paged append/finalize) addresses pages in 64 bits.

An MI355X holds 288 GB, so a serving pool of INT8 pages easily passes the
2**31 bytes (131072 INT8 pages, 65536 FP16 pages at Hkv = 8) where a 32-bit
offset would wrap.  Each test puts a small problem's pages at ids past
that (INT8 ids from 262144: K byte offsets from 4 GiB; FP16 ids from
131072: from 4 GiB), runs the same call on the compact pools and on the
large ones, and requires bit-identical results; the compact results are
pinned against the oracle as in the other tests.  About 18 GB of device
memory, allocated once for the module and never initialised beyond the
pages the tables name."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import assert_bit_equal, cpu, fp16_parity, max_abs, oracle_decode

pytestmark = pytest.mark.gpu

INT8_POOL = 270_000    # 16 KiB of K codes per page: 4.4 GB per pool
FP16_POOL = 140_000    # 32 KiB of K per page: 4.6 GB per pool
INT8_FIRST = 262_144   # first id past 4 GiB of INT8 codes
FP16_FIRST = 131_072   # first id past 4 GiB of FP16 pages


@pytest.fixture(scope="module")
def pools(cuda):
    print(f"large pools: {INT8_POOL} INT8 pages, {FP16_POOL} FP16 pages", flush=True)
    p = {"k_codes": torch.empty(INT8_POOL, 16, 8, 128, dtype=torch.int8, device=cuda),
         "v_codes": torch.empty(INT8_POOL, 16, 8, 128, dtype=torch.int8, device=cuda),
         "k_scale": torch.empty(INT8_POOL, 8, dtype=torch.float16, device=cuda),
         "v_scale": torch.empty(INT8_POOL, 8, dtype=torch.float16, device=cuda),
         "exact_k": torch.empty(FP16_POOL, 16, 8, 128, dtype=torch.float16, device=cuda),
         "exact_v": torch.empty(FP16_POOL, 16, 8, 128, dtype=torch.float16, device=cuda)}
    yield p
    p.clear()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _high_ids(count, first, pool, stride, device):
    """``count`` distinct ids in [first, pool), spread by a stride coprime to the span."""
    ids = first + (torch.arange(count, dtype=torch.int64) * stride) % (pool - first)
    assert ids.unique().numel() == count
    return ids.to(device)


@pytest.fixture(scope="module")
def placed(cuda, pools):
    """A B3 workload (INT8 histories of 97, 203 and 5 pages, a 16-page FP16
    ring each) stored compactly and again at high ids of the large pools."""
    from pagegauge_amd import workloads

    w = workloads.build_decode_workload([16 * (16 + 97), 16 * (16 + 203), 16 * (16 + 5)],
                                        20261201, device=cuda, tail_tokens=256)
    w.tail_last_page_len = torch.tensor([16, 9, 1], dtype=torch.int32, device=cuda)
    old_ids = _high_ids(w.k_codes.shape[0], INT8_FIRST, INT8_POOL, 41, cuda)
    tail_ids = _high_ids(w.tail_k.shape[0], FP16_FIRST, FP16_POOL, 13, cuda)
    for name, src, ids in (("k_codes", w.k_codes, old_ids), ("v_codes", w.v_codes, old_ids),
                           ("k_scale", w.k_scale, old_ids), ("v_scale", w.v_scale, old_ids),
                           ("exact_k", w.tail_k, tail_ids), ("exact_v", w.tail_v, tail_ids)):
        pools[name][ids] = src
    torch.cuda.synchronize()
    big_old = old_ids[w.old_indices.long()].to(torch.int32)
    big_tail = tail_ids[w.tail_indices.long()].to(torch.int32)
    assert int(big_old.min()) >= INT8_FIRST and int(big_tail.min()) >= FP16_FIRST
    return w, big_old, big_tail


@pytest.mark.parametrize("split", [None, 5])
def test_segmented_decode_on_pools_past_4gib(cuda, pools, placed, split):
    from pagegauge_amd import decode

    w, big_old, big_tail = placed
    print(f"large-pool segmented decode split={split}", flush=True)
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=cuda)
    results = []
    for old_idx, tail_idx, k, v, ks, vs, tk, tv in (
            (w.old_indices, w.tail_indices, w.k_codes, w.v_codes, w.k_scale, w.v_scale, w.tail_k,
             w.tail_v),
            (big_old, big_tail, pools["k_codes"], pools["v_codes"], pools["k_scale"],
             pools["v_scale"], pools["exact_k"], pools["exact_v"])):
        dec = decode.PageGaugeSegmentedDecode(ws)
        dec.plan(w.old_indptr, old_idx, w.old_last_page_len, w.tail_indptr, tail_idx,
                 w.tail_last_page_len, fixed_split_size=split)
        out, lse = dec.run(w.query, (k, v), ks, vs, (tk, tv), w.value_center, return_lse=True)
        torch.cuda.synchronize()
        results.append((out.clone(), lse.clone()))
    (out_c, lse_c), (out_b, lse_b) = results
    assert torch.equal(out_b, out_c) and torch.equal(lse_b, lse_c)
    ref_out, ref_lse, ref64 = oracle_decode(w)
    par = fp16_parity(out_c, ref_out, ref64)
    print(f"  {par} lse {max_abs(lse_c, ref_lse):.2e}", flush=True)
    assert par["ok"] and max_abs(lse_c, ref_lse) <= 2e-3


def _unified(w, old_idx, tail_idx, device):
    old_ptr, tail_ptr = w.old_indptr.tolist(), w.tail_indptr.tolist()
    old_idx, tail_idx = old_idx.cpu(), tail_idx.cpu()
    rows, indptr, old_len = [], [0], []
    for b in range(w.batch):
        rows += [old_idx[old_ptr[b]:old_ptr[b + 1]], tail_idx[tail_ptr[b]:tail_ptr[b + 1]]]
        indptr.append(indptr[-1] + old_ptr[b + 1] - old_ptr[b] + tail_ptr[b + 1] - tail_ptr[b])
        old_len.append(16 * (old_ptr[b + 1] - old_ptr[b]))
    return (torch.tensor(indptr, dtype=torch.int32), torch.cat(rows).to(device),
            torch.tensor(old_len, dtype=torch.int32, device=device))


def test_heterogeneous_decode_on_pools_past_4gib(cuda, pools, placed):
    from pagegauge_amd import decode

    w, big_old, big_tail = placed
    print("large-pool heterogeneous decode", flush=True)
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=cuda)
    outs = []
    for old_idx, tail_idx, k, v, ks, vs, tk, tv in (
            (w.old_indices, w.tail_indices, w.k_codes, w.v_codes, w.k_scale, w.v_scale, w.tail_k,
             w.tail_v),
            (big_old, big_tail, pools["k_codes"], pools["v_codes"], pools["k_scale"],
             pools["v_scale"], pools["exact_k"], pools["exact_v"])):
        indptr, unified, old_kv_len = _unified(w, old_idx, tail_idx, cuda)
        het = decode.make_heterogeneous_page_gauge_wrapper(None, ws)
        het.plan(indptr, unified, w.tail_last_page_len, 32, 8, 128, 16, exact_tail_pages_hint=16)
        out = het.run(w.query, (k, v), ks, vs, tk, tv, old_kv_len, w.value_center)
        torch.cuda.synchronize()
        outs.append(out.clone())
    assert torch.equal(outs[1], outs[0])
    ref_out, _, ref64 = oracle_decode(w)
    assert fp16_parity(outs[0], ref_out, ref64)["ok"]


def test_exact_tail_merge_on_pools_past_4gib(cuda, pools, placed):
    from pagegauge_amd import runtime

    ext = runtime.load_append_extension()
    w, _, big_tail = placed
    print("large-pool exact tail merge", flush=True)
    gen = torch.Generator().manual_seed(3)
    old_out = torch.randn(w.batch, 32, 128, generator=gen).to(torch.float16).to(cuda)
    old_lse = (torch.randn(w.batch, 32, generator=gen) * 4 + 10).to(cuda)
    results = []
    for idx, tk, tv in ((w.tail_indices, w.tail_k, w.tail_v),
                        (big_tail, pools["exact_k"], pools["exact_v"])):
        out, lse = old_out.clone(), old_lse.clone()
        ext.exact_tail_merge_center(w.query, tk, tv, idx, w.tail_last_page_len, out, lse,
                                    w.value_center, w.sm_scale)
        torch.cuda.synchronize()
        results.append((out, lse))
    assert torch.equal(results[1][0], results[0][0]) and torch.equal(results[1][1], results[0][1])


def _rand(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.float16)


def test_slots_append_finalize_on_pools_past_4gib(cuda, pools):
    """K2 through serving slots: rows written into the last exact pages of
    the pool (4.6 GB in), completed pages finalized into its last code pages
    (4.4 GB in); positions 15 and 47 complete a page, 70 does not."""
    from pagegauge_amd import runtime

    ext = runtime.load_append_extension()
    print("large-pool slots append/finalize", flush=True)
    gen = torch.Generator().manual_seed(20261202)
    batch = 3
    positions = torch.tensor([15, 47, 70], dtype=torch.int32, device=cuda)
    q, k, v = _rand(gen, batch, 32, 128), _rand(gen, batch, 8, 128), _rand(gen, batch, 8, 128)
    cos, sin = _rand(gen, 80, 128), _rand(gen, 80, 128)
    kc, vc = _rand(gen, batch, 8, 128, scale=0.1), _rand(gen, batch, 8, 128, scale=0.1)
    ring_k, ring_v = _rand(gen, batch, 16, 8, 128, scale=0.5), _rand(gen, batch, 16, 8, 128, scale=0.5)
    exact_ids = torch.arange(FP16_POOL - 1, FP16_POOL - 1 - batch, -1, device=cuda)
    code_ids = torch.arange(INT8_POOL - 1, INT8_POOL - 1 - batch, -1, device=cuda)
    small = [ring_k.to(cuda), ring_v.to(cuda),
             torch.zeros(batch, 16, 8, 128, dtype=torch.int8, device=cuda),
             torch.zeros(batch, 16, 8, 128, dtype=torch.int8, device=cuda),
             torch.zeros(batch, 8, dtype=torch.float16, device=cuda),
             torch.zeros(batch, 8, dtype=torch.float16, device=cuda)]
    big = [pools[n] for n in ("exact_k", "exact_v", "k_codes", "v_codes", "k_scale", "v_scale")]
    for t, src, ids in zip(big, small, (exact_ids, exact_ids) + (code_ids,) * 4):
        t[ids] = src
    host = [cpu(t).copy() for t in small]
    d = [t.to(cuda) for t in (q, k, v, cos, sin, kc, vc)]
    rq_small = torch.zeros(batch, 32, 128, dtype=torch.float16, device=cuda)
    rq_big = torch.zeros_like(rq_small)
    local = torch.arange(batch, dtype=torch.int32, device=cuda)
    ext.rope_append_page_gauge_slots(*d[:5], positions, local, local, d[5], d[6], rq_small, *small)
    ext.rope_append_page_gauge_slots(*d[:5], positions, exact_ids.to(torch.int32),
                                     code_ids.to(torch.int32), d[5], d[6], rq_big, *big)
    torch.cuda.synchronize()
    hq = np.zeros((batch, 32, 128), np.float16)
    oracle.rope_append_page_gauge_slots(q.numpy(), k.numpy(), v.numpy(), cos.numpy(), sin.numpy(),
                                        cpu(positions), np.arange(batch), np.arange(batch),
                                        kc.numpy(), vc.numpy(), hq, *host)
    assert torch.equal(rq_big, rq_small)
    assert_bit_equal(rq_small, hq, "rotated query")
    names = ("exact K", "exact V", "K codes", "V codes", "K scales", "V scales")
    for t, s_t, h, ids, name in zip(big, small, host, (exact_ids, exact_ids) + (code_ids,) * 4,
                                    names):
        assert torch.equal(t[ids], s_t), name
        assert_bit_equal(s_t, h, name)
    assert int((host[2] != 0).any(axis=(1, 2, 3)).sum()) == 2      # two pages finalized


def test_paged_append_finalize_on_pools_past_2gib(cuda, pools):
    """The paged append/finalize (one id for the exact page, its codes and
    scales): pages at the end of a 140000-page pool, 4.6 GB into the FP16
    pages and 2.3 GB into the codes."""
    from pagegauge_amd import update

    print("large-pool paged append/finalize", flush=True)
    gen = torch.Generator().manual_seed(20261203)
    batch = 3
    k, v = _rand(gen, batch, 8, 128), _rand(gen, batch, 8, 128)
    kc, vc = _rand(gen, 8, 128, scale=0.1), _rand(gen, 8, 128, scale=0.1)
    ring_k, ring_v = _rand(gen, batch, 16, 8, 128, scale=0.5), _rand(gen, batch, 16, 8, 128, scale=0.5)
    offsets = torch.tensor([15, 15, 7], dtype=torch.int32, device=cuda)
    ids = torch.arange(FP16_POOL - 4, FP16_POOL - 4 - batch, -1, device=cuda)
    small = [ring_k.to(cuda), ring_v.to(cuda),
             torch.zeros(batch, 16, 8, 128, dtype=torch.int8, device=cuda),
             torch.zeros(batch, 16, 8, 128, dtype=torch.int8, device=cuda),
             torch.zeros(batch, 8, dtype=torch.float16, device=cuda),
             torch.zeros(batch, 8, dtype=torch.float16, device=cuda)]
    big = [pools["exact_k"], pools["exact_v"], pools["k_codes"][:FP16_POOL],
           pools["v_codes"][:FP16_POOL], pools["k_scale"][:FP16_POOL], pools["v_scale"][:FP16_POOL]]
    for t, src in zip(big, small):
        t[ids] = src
    host = [cpu(t).copy() for t in small]
    dk, dv, dkc, dvc = (t.to(cuda) for t in (k, v, kc, vc))
    update.append_finalize_page_gauge(dk, dv, dkc, dvc, *small,
                                      torch.arange(batch, dtype=torch.int32, device=cuda), offsets)
    update.append_finalize_page_gauge(dk, dv, dkc, dvc, *big, ids.to(torch.int32), offsets)
    torch.cuda.synchronize()
    oracle.append_finalize_page_gauge(k.numpy(), v.numpy(), kc.numpy(), vc.numpy(), *host,
                                      np.arange(batch), cpu(offsets))
    names = ("exact K", "exact V", "K codes", "V codes", "K scales", "V scales")
    for t, s_t, h, name in zip(big, small, host, names):
        assert torch.equal(t[ids], s_t), name
        assert_bit_equal(s_t, h, name)
    assert int((host[2] != 0).any(axis=(1, 2, 3)).sum()) == 2
