"""GPU parity of the paged-decode kernels against the float64 oracle.

Tolerance: attention outputs max-abs <= 2e-3 in FP16
units; base-2 LSE max-abs <= 2e-3.  Cases cover the segmented INT8+tail
decode (configs 1-3 at reduced and full size), the INT8-only and FP16
wrappers at every split, partial last pages, empty segments and the
boundary cases of diagnostics/benchmark_heterogeneous_fa2_correctness.py:63-73.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import cpu, max_abs, oracle_decode

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-3
LSE_TOL = 2e-3


@pytest.fixture(scope="module")
def workspace(cuda):
    return torch.empty(64 << 20, dtype=torch.uint8, device=cuda)


def _segmented(w, workspace, split=None, tail_split=None, center=True):
    from pagegauge_amd import decode

    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, fixed_split_size=split, tail_split_size=tail_split)
    out, lse = dec.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                       w.value_center if center else None, return_lse=True)
    torch.cuda.synchronize()
    return out, lse, dec


@pytest.mark.parametrize("lengths,split", [
    ([4096], None),             # config 1 shape
    ([4096], 1), ([4096], 3), ([4096], 4), ([4096], 5), ([4096], 240),
    ([272, 2048, 512], None),   # ragged, shortest with a single history page
    ([4096 + 16 * 7, 1024], 7),
    ([8192], 1),                # 496 + 16 one-page items: a one-request plan in two rounds
    ([8192 + 16 * 5, 2048], 1), # the same over two requests (work list in dispatch order)
])
def test_segmented_decode_matches_oracle(cuda, workspace, lengths, split):
    from pagegauge_amd import workloads

    w = workloads.build_decode_workload(lengths, seed=20260840, device=cuda)
    out, lse, _ = _segmented(w, workspace, split=split)
    ref_out, ref_lse, _ = oracle_decode(w)
    assert max_abs(out, ref_out) <= OUT_TOL
    assert max_abs(lse, ref_lse) <= LSE_TOL


@pytest.mark.parametrize("seed", [20260840, 20260841, 20260842])
def test_b8_ragged_config3(cuda, workspace, seed):
    from pagegauge_amd import workloads

    w = workloads.b8_ragged(seed, device=cuda)
    out, lse, dec = _segmented(w, workspace)
    ref_out, ref_lse, _ = oracle_decode(w)
    assert max_abs(out, ref_out) <= OUT_TOL
    assert max_abs(lse, ref_lse) <= LSE_TOL
    assert dec.num_work_items >= 8


@pytest.mark.parametrize("lengths", [[28672] * 4, [65536]])
def test_medium_plans_with_long_items(cuda, workspace, lengths):
    """Medium-regime plans up to 30 weighted pages per CU: 112-120 items of
    up to 64 pages (16 groups per wave, the PV accumulators' exactness
    bound), each over two half-height workgroups."""
    from pagegauge_amd import workloads

    w = workloads.build_decode_workload(lengths, seed=20260841, device=cuda)
    out, lse, dec = _segmented(w, workspace)
    plan = dec._state.plan
    print("medium", lengths[0], len(lengths), plan.num_items, plan.waves_per_block, flush=True)
    assert plan.waves_per_block == 4 and 112 <= plan.num_items <= 120
    ref_out, ref_lse, _ = oracle_decode(w)
    assert max_abs(out, ref_out) <= OUT_TOL
    assert max_abs(lse, ref_lse) <= LSE_TOL


def test_large_plan_one_request(cuda, workspace):
    """One request past 30 weighted pages per CU (128K tokens: 8192 INT8
    pages + the 16-page ring): the large plan's one-round items in 8-wave
    workgroups, described in closed form (no work-item loads)."""
    from pagegauge_amd import workloads

    w = workloads.build_decode_workload([131072 + 256], seed=20260842, device=cuda)
    out, lse, dec = _segmented(w, workspace)
    plan = dec._state.plan
    print("large B1", plan.num_items, plan.waves_per_block, plan.closed_form, flush=True)
    assert plan.waves_per_block == 8 and plan.closed_form == 1 and plan.num_items <= 256
    ref_out, ref_lse, _ = oracle_decode(w)
    assert max_abs(out, ref_out) <= OUT_TOL
    assert max_abs(lse, ref_lse) <= LSE_TOL


@pytest.mark.parametrize("flat,code", [("query", 127), ("query", -127), ("keys", 127)])
def test_pv_digits_of_64_page_items_at_the_accumulator_bound(cuda, workspace, flat, code):
    """Adversarial 64-page INT8 items (16 PV groups without a fold).

    Equal scores (a zero query, or all-zero K codes) keep the running max
    flat, so the PV accumulators sum all 16 groups before they are folded.
    Every V code is +-127 and every V page scale is 1040/1024 * 2^-7: the
    probability's fixed point is then 0x208000, whose middle radix-256
    digit is -128 on every token, so the middle accumulator row reaches
    16 * 64 * 128 * 127 = 16,646,144 in magnitude, and 256 times that passes
    2^31.  The result must still match the oracle."""
    from pagegauge_amd import workloads

    w = workloads.build_decode_workload([2 * 64 * 16 + 256], seed=20260845, device=cuda)
    if flat == "query":
        w.query.zero_()
    else:
        w.k_codes.zero_()
    w.v_codes.fill_(code)
    w.v_scale.fill_(1040 / 1024 * 2 ** -7)
    assert float(w.v_scale[0, 0]) == 1040 / 1024 * 2 ** -7
    out, lse, dec = _segmented(w, workspace, split=64)
    assert dec.split_pages == 64 and dec._state.plan.num_items_primary == 2
    ref_out, ref_lse, _ = oracle_decode(w)
    print("pv64", flat, code, max_abs(out, ref_out), flush=True)
    assert max_abs(out, ref_out) <= OUT_TOL
    assert max_abs(lse, ref_lse) <= LSE_TOL


def test_b1_49k_config2_full_size(cuda, workspace):
    from pagegauge_amd import workloads

    w = workloads.b1_49k(20260840, device=cuda)
    assert int(w.old_indices.numel()) == 3056 and int(w.tail_indices.numel()) == 16
    out, lse, dec = _segmented(w, workspace)
    ref_out, ref_lse, _ = oracle_decode(w)
    assert max_abs(out, ref_out) <= OUT_TOL
    assert max_abs(lse, ref_lse) <= LSE_TOL
    # size-independent property: results do not depend on the split choice
    out2, lse2, _ = _segmented(w, workspace, split=48, tail_split=16)
    assert max_abs(out, out2) <= OUT_TOL
    assert max_abs(lse, lse2) <= 1e-3


def test_int8_wrapper_matches_oracle_without_center(cuda, workspace):
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload([2048, 1024 + 256], seed=11, device=cuda)
    wrapper = decode.make_page_gauge_wrapper(None, workspace)
    for split in (None, 1, 2, 7, 16):
        wrapper.plan(w.old_indptr, w.old_indices, w.old_last_page_len, 32, 8, 128, 16,
                     pos_encoding_mode="NONE", q_data_type=torch.float16,
                     kv_data_type=torch.int8, o_data_type=torch.float16,
                     sm_scale=128 ** -0.5, fixed_split_size=split)
        out = torch.empty_like(w.query)
        lse = torch.empty(w.batch, 32, dtype=torch.float32, device=cuda)
        wrapper.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, 128 ** -0.5, out=out,
                    lse=lse, return_lse=True)
        torch.cuda.synchronize()
        ref_out, ref_lse, _ = oracle_decode(w, with_tail=False, with_center=False)
        assert max_abs(out, ref_out) <= OUT_TOL, split
        assert max_abs(lse, ref_lse) <= LSE_TOL, split


def test_partial_last_page_is_masked(cuda, workspace):
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload([1024], seed=3, device=cuda)
    for last in (1, 7, 15):
        w.old_last_page_len.fill_(last)
        w.tail_last_page_len.fill_(16 - last)
        out, lse, _ = _segmented(w, workspace, split=5, tail_split=3)
        ref_out, ref_lse, _ = oracle_decode(w)
        assert max_abs(out, ref_out) <= OUT_TOL
        assert max_abs(lse, ref_lse) <= LSE_TOL
    # last_page_len is re-read on every run: advance it without re-planning
    wrapper = decode.make_page_gauge_wrapper(None, workspace)
    w.old_last_page_len.fill_(16)
    wrapper.plan(w.old_indptr, w.old_indices, w.old_last_page_len, 32, 8, 128, 16,
                 kv_data_type=torch.int8, fixed_split_size=4)
    for last in (16, 9, 2):
        w.old_last_page_len.fill_(last)
        out = wrapper.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale)
        torch.cuda.synchronize()
        ref_out, _, _ = oracle_decode(w, with_tail=False, with_center=False)
        assert max_abs(out, ref_out) <= OUT_TOL


def test_fp16_wrapper_same_way_kernel(cuda, workspace):
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload([2048, 768], seed=5, device=cuda, with_fp16_copy=True)
    wrapper = decode.BatchDecodeWithPagedKVCacheWrapper(workspace, "NHD")
    for split in (None, 1, 3, 8):
        wrapper.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 32, 8, 128, 16,
                     kv_data_type=torch.float16, fixed_split_size=split)
        out, lse = wrapper.run(w.query, (w.fp16_k, w.fp16_v), return_lse=True)
        torch.cuda.synchronize()
        ref_out, ref_lse, _ = oracle.decode(cpu(w.query), cpu(w.fp16_k), cpu(w.fp16_v),
                                            cpu(w.fp16_indptr), cpu(w.fp16_indices),
                                            cpu(w.fp16_last_page_len), w.sm_scale)
        assert max_abs(out, ref_out) <= OUT_TOL, split
        assert max_abs(lse, ref_lse) <= LSE_TOL, split


def test_segmented_equals_int8_fp16_merge_center(cuda, workspace):
    """run_affine composition: INT8 wrapper + FP16 tail + merge_state + center."""
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload([3072], seed=9, device=cuda)
    fused, fused_lse, _ = _segmented(w, workspace)
    ws2 = torch.empty(8 << 20, dtype=torch.uint8, device=cuda)
    int8 = decode.make_page_gauge_wrapper(None, ws2)
    int8.plan(w.old_indptr, w.old_indices, w.old_last_page_len, 32, 8, 128, 16,
              kv_data_type=torch.int8)
    out, lse = int8.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, w.sm_scale,
                        return_lse=True)
    ws3 = torch.empty(8 << 20, dtype=torch.uint8, device=cuda)
    tail = decode.BatchDecodeWithPagedKVCacheWrapper(ws3)
    tail.plan(w.tail_indptr, w.tail_indices, w.tail_last_page_len, 32, 8, 128, 16,
              kv_data_type=torch.float16)
    tout, tlse = tail.run(w.query, (w.tail_k, w.tail_v), return_lse=True)
    decode.merge_state_in_place(out, lse, tout, tlse)
    out += w.value_center.repeat_interleave(4, dim=1)
    torch.cuda.synchronize()
    assert max_abs(out, fused) <= OUT_TOL
    assert max_abs(lse, fused_lse) <= 1e-3


def test_merge_state_in_place_matches_oracle(cuda):
    from pagegauge_amd import decode

    gen = torch.Generator().manual_seed(2)
    v = (torch.randn(5, 32, 128, generator=gen) * 0.3).half()
    vo = (torch.randn(5, 32, 128, generator=gen) * 0.3).half()
    s = torch.randn(5, 32, generator=gen) * 3
    so = torch.randn(5, 32, generator=gen) * 3
    s[0, 0] = float("-inf")
    mask = torch.tensor([1, 0, 1, 1, 0], dtype=torch.bool)
    want_v, want_s = oracle.merge_state_in_place(v.numpy(), s.numpy(), vo.numpy(), so.numpy(),
                                                 mask.numpy())
    dv, ds = v.cuda(), s.cuda()
    decode.merge_state_in_place(dv, ds, vo.cuda(), so.cuda(), mask.cuda())
    torch.cuda.synchronize()
    assert max_abs(dv, want_v) <= 1e-3
    assert max_abs(ds, want_s) <= 1e-4


@pytest.mark.parametrize("old_pages,total_tokens", [
    (16, 256),   # old only (no tail tokens)
    (0, 1), (0, 15), (0, 16),   # exact only
    (1, 17), (1, 31), (1, 32), (9, 176), (9, 191),
])
def test_boundary_cases_of_reference_fixture(cuda, workspace, old_pages, total_tokens):
    """The 9 CASES of diagnostics/benchmark_heterogeneous_fa2_correctness.py:63-73."""
    from pagegauge_amd import decode

    gen = torch.Generator().manual_seed(20260816)
    batch = 2
    tail_tokens = total_tokens - 16 * old_pages
    tail_pages = (tail_tokens + 15) // 16
    q = (torch.randn(batch, 32, 128, generator=gen) * 0.35).half().cuda()
    k_codes = torch.randint(-127, 128, (batch * max(old_pages, 1), 16, 8, 128), generator=gen,
                            dtype=torch.int8).cuda()
    v_codes = torch.randint(-127, 128, k_codes.shape, generator=gen, dtype=torch.int8).cuda()
    k_scale = (torch.rand(k_codes.shape[0], 8, generator=gen) * 1e-3 + 1e-4).half().cuda()
    v_scale = (torch.rand(k_codes.shape[0], 8, generator=gen) * 1e-3 + 1e-4).half().cuda()
    ring = max(tail_pages, 1) * batch
    tail_k = (torch.randn(ring, 16, 8, 128, generator=gen) * 0.08).half().cuda()
    tail_v = (torch.randn(ring, 16, 8, 128, generator=gen) * 0.08).half().cuda()
    center = (torch.randn(batch, 8, 128, generator=gen) * 0.025).half().cuda()
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device="cuda")  # noqa: E731
    old_indptr = i32([0, old_pages, 2 * old_pages])
    old_indices = i32(list(reversed(range(batch * old_pages)))) if old_pages else i32([0])
    tail_indptr = i32([0, tail_pages, 2 * tail_pages])
    tail_indices = i32(list(range(batch * tail_pages))) if tail_pages else i32([0])
    last_tail = (tail_tokens - 1) % 16 + 1 if tail_pages else 16
    old_last = i32([16] * batch)
    tail_last = i32([last_tail] * batch)
    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(old_indptr, old_indices, old_last, tail_indptr, tail_indices, tail_last,
             fixed_split_size=2, tail_split_size=1)
    out, lse = dec.run(q, (k_codes, v_codes), k_scale, v_scale, (tail_k, tail_v), center,
                       return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, _ = oracle.decode(
        cpu(q), cpu(k_codes), cpu(v_codes), cpu(old_indptr), cpu(old_indices), cpu(old_last),
        128 ** -0.5, k_scale=cpu(k_scale), v_scale=cpu(v_scale), tail_k=cpu(tail_k),
        tail_v=cpu(tail_v), tail_indptr=cpu(tail_indptr), tail_indices=cpu(tail_indices),
        tail_last_page_len=cpu(tail_last), value_center=cpu(center))
    assert max_abs(out, ref_out) <= OUT_TOL
    assert max_abs(lse, ref_lse) <= LSE_TOL


def test_empty_request_gives_center_and_neg_inf_lse(cuda, workspace):
    from pagegauge_amd import decode

    q = torch.randn(1, 32, 128, device=cuda).half()
    codes = torch.zeros(1, 16, 8, 128, dtype=torch.int8, device=cuda)
    scale = torch.ones(1, 8, dtype=torch.float16, device=cuda)
    ring = torch.zeros(1, 16, 8, 128, dtype=torch.float16, device=cuda)
    center = torch.randn(1, 8, 128, device=cuda).half()
    z = torch.zeros(2, dtype=torch.int32, device=cuda)
    idx = torch.zeros(1, dtype=torch.int32, device=cuda)
    last = torch.full((1,), 16, dtype=torch.int32, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(z, idx, last, z, idx, last)
    out, lse = dec.run(q, (codes, codes), scale, scale, (ring, ring), center, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, center.repeat_interleave(4, dim=1))
    assert bool(torch.isneginf(lse).all())


def test_bound_timed_call_equals_plain_call(cuda, workspace):
    """pg_decode_run_timed (dispatch-stamped events) computes exactly what
    pg_decode_run does, and its events measure a positive GPU time."""
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload([4096, 1024], seed=20260844, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len)
    outs = []
    for timed in (False, True):
        out = torch.full_like(w.query, float("nan"))
        lse = torch.full((w.batch, 32), float("nan"), dtype=torch.float32, device=cuda)
        bound = dec.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                         (w.tail_k, w.tail_v), w.value_center, out=out, lse=lse)
        if timed:
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            stop.record()
            torch.cuda.synchronize()
            bound.timed(start.cuda_event, stop.cuda_event)
            torch.cuda.synchronize()
            assert start.elapsed_time(stop) > 0.0
        else:
            bound()
            torch.cuda.synchronize()
        outs.append((cpu(out), cpu(lse)))
    assert np.array_equal(outs[0][0].view(np.uint16), outs[1][0].view(np.uint16))
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))


def test_bound_decode_refuses_to_run_after_a_new_plan(cuda, workspace):
    """A bound call carries the pointers of the tables it was bound to; once
    its wrapper plans other tables into the workspace it must not launch."""
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload([4096], seed=20260842, device=cuda)
    w2 = workloads.build_decode_workload([2048, 1024], seed=20260843, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len)
    out = torch.empty_like(w.query)
    bound = dec.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                     w.value_center, out=out)
    bound()
    dec.plan(w2.old_indptr, w2.old_indices, w2.old_last_page_len, w2.tail_indptr,
             w2.tail_indices, w2.tail_last_page_len)
    for call in (bound, bound.partial, bound.combine):
        with pytest.raises(RuntimeError, match="planned again"):
            call()
    out2 = torch.empty_like(w2.query)
    dec.bind(w2.query, (w2.k_codes, w2.v_codes), w2.k_scale, w2.v_scale, (w2.tail_k, w2.tail_v),
             w2.value_center, out=out2)()
    torch.cuda.synchronize()
    ref_out, _, _ = oracle_decode(w2)
    assert max_abs(out2, ref_out) <= OUT_TOL
