"""The VALU alternative of the INT8 QK contraction (``python -m
pagegauge_amd.build --variant qk_valu``) computes the same integer digit dot
products as the product's i8 MFMA, so its decode outputs must be bit-identical
to the product's on the same plan and inputs.  Skipped when the alternative
build is absent or older than the sources (it is built on request only)."""

from __future__ import annotations

import ctypes

import pytest
import torch

from pagegauge_amd import _capi, build, decode, workloads

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def valu_library():
    if not build.variant_is_current("qk_valu"):
        pytest.skip("qk_valu alternative build absent or stale "
                    "(python -m pagegauge_amd.build --variant qk_valu)")
    return _capi.load_library(build.variant_library("qk_valu"))


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


@pytest.mark.parametrize("lengths,split", [([8192], None), ([720, 4096, 1008], 7), ([2048], 64)])
def test_valu_qk_is_bit_identical_to_the_mfma(cuda, valu_library, lengths, split):
    w = workloads.build_decode_workload(lengths, 20260840, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(torch.empty(16 << 20, dtype=torch.uint8, device=cuda))
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, fixed_split_size=split)
    out, lse = dec.run(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                       w.value_center, return_lse=True)
    out2, lse2 = torch.full_like(out, float("nan")), torch.full_like(lse, float("nan"))
    _run(valu_library, dec, w, out2, lse2)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
