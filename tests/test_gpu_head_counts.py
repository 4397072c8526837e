"""Paged decode with KV head counts other than Mistral's 8 (GQA group 4:
Hq = 4 * Hkv).  The kernels specialise Hkv = 8 (a compile-time row stride)
and take every other count through the general path (row stride
Hkv * 128 at run time, workgroups of 1, 2, 4 or 8 KV-head waves); these
cases run that path: the segmented INT8 + FP16-tail decode, the INT8-only
wrapper and the FP16 same-way wrapper, against the float64 oracle (out and
lse max-abs <= 2e-3), at the planner's split and a fixed one.

The caches are the seeded 8-head workload cut to Hkv heads (1, 2, 4), or
two copies side by side for 16 heads (the second with its heads reversed
and its codes negated, so the two halves differ)."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import cpu, max_abs, oracle

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module")
def workspace(cuda):
    return torch.empty(64 << 20, dtype=torch.uint8, device=cuda)


def _heads(t, hkv, axis, negate=False):
    """Cut ``t`` to ``hkv`` heads along ``axis`` (8 heads), or widen it to 16."""
    if hkv <= 8:
        return t.narrow(axis, 0, hkv).contiguous()
    other = t.flip(axis)
    if negate:
        other = -other
    return torch.cat((t, other), dim=axis).contiguous()


@pytest.fixture(scope="module", params=[1, 2, 4, 16])
def case(request, cuda):
    from pagegauge_amd import workloads

    hkv = request.param
    w = workloads.build_decode_workload([2048 + 256, 1024 + 256, 512 + 256], 20260860 + hkv,
                                        device=cuda, with_fp16_copy=True)
    q = _heads(w.query.view(w.batch, 8, 4, 128), hkv, 1).view(w.batch, 4 * hkv, 128)
    data = {
        "hkv": hkv, "w": w, "q": q.contiguous(),
        "k_codes": _heads(w.k_codes, hkv, 2, negate=True),
        "v_codes": _heads(w.v_codes, hkv, 2, negate=True),
        "k_scale": _heads(w.k_scale, hkv, 1), "v_scale": _heads(w.v_scale, hkv, 1),
        "tail_k": _heads(w.tail_k, hkv, 2), "tail_v": _heads(w.tail_v, hkv, 2),
        "center": _heads(w.value_center, hkv, 1),
        "fp16_k": _heads(w.fp16_k, hkv, 2), "fp16_v": _heads(w.fp16_v, hkv, 2),
    }
    return data


@pytest.mark.parametrize("split", [None, 5])
def test_segmented_decode_any_kv_head_count(case, workspace, split):
    from pagegauge_amd import decode

    w, hkv = case["w"], case["hkv"]
    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, num_qo_heads=4 * hkv, num_kv_heads=hkv,
             fixed_split_size=split)
    out, lse = dec.run(case["q"], (case["k_codes"], case["v_codes"]), case["k_scale"],
                       case["v_scale"], (case["tail_k"], case["tail_v"]), case["center"],
                       return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, _ = oracle.decode(
        cpu(case["q"]), cpu(case["k_codes"]), cpu(case["v_codes"]), cpu(w.old_indptr),
        cpu(w.old_indices), cpu(w.old_last_page_len), w.sm_scale, k_scale=cpu(case["k_scale"]),
        v_scale=cpu(case["v_scale"]), tail_k=cpu(case["tail_k"]), tail_v=cpu(case["tail_v"]),
        tail_indptr=cpu(w.tail_indptr), tail_indices=cpu(w.tail_indices),
        tail_last_page_len=cpu(w.tail_last_page_len), value_center=cpu(case["center"]))
    print(f"Hkv {hkv} split {split}: {dec.num_work_items} items, "
          f"{int(dec._state.plan.waves_per_block)} waves per workgroup", flush=True)
    assert max_abs(out, ref_out) <= TOL and max_abs(lse, ref_lse) <= TOL


def test_int8_and_fp16_wrappers_any_kv_head_count(case, workspace):
    from pagegauge_amd import decode

    w, hkv = case["w"], case["hkv"]
    wrapper = decode.make_page_gauge_wrapper(None, workspace)
    wrapper.plan(w.old_indptr, w.old_indices, w.old_last_page_len, 4 * hkv, hkv, 128, 16,
                 kv_data_type=torch.int8, fixed_split_size=7)
    out, lse = wrapper.run(case["q"], (case["k_codes"], case["v_codes"]), case["k_scale"],
                           case["v_scale"], return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, _ = oracle.decode(
        cpu(case["q"]), cpu(case["k_codes"]), cpu(case["v_codes"]), cpu(w.old_indptr),
        cpu(w.old_indices), cpu(w.old_last_page_len), w.sm_scale, k_scale=cpu(case["k_scale"]),
        v_scale=cpu(case["v_scale"]))
    assert max_abs(out, ref_out) <= TOL and max_abs(lse, ref_lse) <= TOL

    fp16 = decode.BatchDecodeWithPagedKVCacheWrapper(workspace, "NHD")
    fp16.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 4 * hkv, hkv, 128, 16,
              kv_data_type=torch.float16)
    out, lse = fp16.run(case["q"], (case["fp16_k"], case["fp16_v"]), return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, _ = oracle.decode(
        cpu(case["q"]), cpu(case["fp16_k"]), cpu(case["fp16_v"]), cpu(w.fp16_indptr),
        cpu(w.fp16_indices), cpu(w.fp16_last_page_len), w.sm_scale)
    assert max_abs(out, ref_out) <= TOL and max_abs(lse, ref_lse) <= TOL
