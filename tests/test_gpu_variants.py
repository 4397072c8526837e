"""Alternative builds of the product (``python -m pagegauge_amd.build
--variant NAME``; built on request only, each kept for a measured design
comparison) must compute the product's decode outputs bit for bit:

* ``qk_valu``: the INT8 QK contraction on the VALU (``v_dot4_i32_i8``) over
  the same integer query digits as the product's i8 MFMA;
* ``default_scheduler``: the same source under LLVM's default scheduler;
* ``interleaved_heads``: an item's workgroups take interleaved KV heads;
* ``full_line_k``: whole-row K loads and a DPP hand-over of the MFMA operand;
* ``trace``, ``trace_conditional_scales``: the phase-trace builds, with and
  without a trace buffer set (with one, every wave of both kernels writes a
  row, checked for the marks' order).

Each variant is skipped when its build is absent or older than the sources."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from pagegauge_amd import _capi, build, decode, workloads

pytestmark = pytest.mark.gpu

CASES = [([8192], None), ([720, 4096, 1008], 7), ([2048], 64), ([16400], None)]


def _variant(name):
    if not build.variant_is_current(name):
        pytest.skip(f"{name} alternative build absent or stale "
                    f"(python -m pagegauge_amd.build --variant {name})")
    return _capi.load_library(build.variant_library(name))


def _run(lib, dec, w, out, lse):
    plan = dec._state.plan
    rc = lib.pg_decode_run(ctypes.byref(plan), w.query.data_ptr(), w.query.stride(0),
                           w.k_codes.data_ptr(), w.v_codes.data_ptr(), w.k_scale.data_ptr(),
                           w.v_scale.data_ptr(), w.old_indices.data_ptr(),
                           w.old_last_page_len.data_ptr(), w.tail_k.data_ptr(), w.tail_v.data_ptr(),
                           w.tail_indices.data_ptr(), w.tail_last_page_len.data_ptr(),
                           w.value_center.data_ptr(), 8 * 128 if w.value_center.dim() == 3 else 0,
                           out.data_ptr(), lse.data_ptr(), w.sm_scale,
                           dec._state.workspace.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.pg_last_error()


def _product_and_plan(cuda, lengths, split):
    w = workloads.build_decode_workload(lengths, 20260840, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(torch.empty(16 << 20, dtype=torch.uint8, device=cuda))
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, fixed_split_size=split)
    out, lse = dec.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                       w.value_center, return_lse=True)
    return w, dec, out, lse


@pytest.mark.parametrize("variant", ["qk_valu", "default_scheduler", "interleaved_heads", "trace",
                                     "trace_conditional_scales", "full_line_k"])
@pytest.mark.parametrize("lengths,split", CASES)
def test_variant_is_bit_identical_to_the_product(cuda, variant, lengths, split):
    lib = _variant(variant)
    w, dec, out, lse = _product_and_plan(cuda, lengths, split)
    out2, lse2 = torch.full_like(out, float("nan")), torch.full_like(lse, float("nan"))
    _run(lib, dec, w, out2, lse2)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(lse, lse2)


@pytest.mark.parametrize("lengths", [[16400], [720, 4096, 1008],
                                     workloads.ragged_lengths(workloads.VALIDATION_SEEDS[0])])
def test_trace_rows_with_the_buffer_set(cuda, lengths):
    """With a trace buffer, the trace build still returns the product's bits,
    and every wave of the partial kernel and (for the four-workgroup combine)
    of the combine kernel writes its row: a known XCD, and marks in the
    order the kernel reaches them (32-bit counter differences, which a wrap
    of s_memrealtime leaves intact).  Shapes: the medium plan (4-wave
    workgroups), a small ragged batch, and config 3's B8 ragged batch (the
    large plan's 8-wave workgroups)."""
    lib = _variant("trace")
    w, dec, out, lse = _product_and_plan(cuda, lengths, None)
    plan = dec._state.plan
    partial_waves = plan.num_items * 8
    combine_waves = w.batch * 32 * 4 * 4
    buf = torch.zeros((partial_waves + combine_waves) * 64, dtype=torch.int32, device=cuda)
    _capi.check(lib.pg_trace_set_buffer(buf.data_ptr(), buf.numel() * 4), "trace")
    try:
        out2, lse2 = torch.full_like(out, float("nan")), torch.full_like(lse, float("nan"))
        _run(lib, dec, w, out2, lse2)
        torch.cuda.synchronize()
    finally:
        _capi.check(lib.pg_trace_set_buffer(None, 0), "trace")
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    rows = buf.view(-1, 64).cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    part, comb = rows[:partial_waves], rows[partial_waves:]
    after = lambda r, a, b: ((r[:, b] - r[:, a]) & 0xFFFFFFFF) < (1 << 31)   # noqa: E731
    assert np.all(part[:, 53] & 0xF < 8) and np.all(part[:, 56] != 100)
    # one row per wave of the grid: every (item, KV head) exactly once
    seen = sorted(int(x) for x in part[:, 55])
    assert seen == sorted((i << 8) | h for i in range(plan.num_items) for h in range(8))
    assert np.all(after(part, 0, 52))                      # start .. end
    int8 = part[:, 56] == 0
    assert int8.any()
    p8 = part[int8]
    assert np.all(after(p8, 0, 1) & after(p8, 1, 2) & after(p8, 2, 4) & after(p8, 4, 52))
    if plan.max_items_per_request > 32 or w.batch * 32 < 512:
        # the four-workgroup combine writes rows (the row kernel does not)
        assert np.all(comb[:, 56] == 100) and np.all(comb[:, 53] & 0xF < 8)
        assert np.all(after(comb, 0, 1) & after(comb, 1, 2) & after(comb, 2, 3)
                      & after(comb, 3, 4) & after(comb, 4, 5))
