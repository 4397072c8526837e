"""The HIP library against the committed golden fixtures (``tests/golden``):
bit-exact for the cache update, within the fp16 tolerance for attention."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import assert_bit_equal, max_abs
from tests.test_golden import load

pytestmark = pytest.mark.gpu

ATOL_OUT = 2e-3       # fp16 output, max-abs
ATOL_LSE = 2e-4       # base-2 lse (reference gate, tests/test_page_gauge_append_extension.py:660)


@pytest.fixture(scope="module")
def ext(cuda):
    from pagegauge_amd import runtime

    return runtime.load_append_extension()


def test_k2_append_fixture_bit_exact(ext, cuda):
    f = load("k2_append")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    batch, hq = f["query"].shape[:2]
    hkv = f["keys"].shape[2]
    ring, code_pages, sink = int(f["ring_pages"]), int(f["code_pages"]), int(f["exact_sink_pages"])
    state = [torch.zeros(batch * ring, 16, hkv, 128, dtype=torch.float16, device=cuda),
             torch.zeros(batch * ring, 16, hkv, 128, dtype=torch.float16, device=cuda),
             torch.zeros(batch * code_pages, 16, hkv, 128, dtype=torch.int8, device=cuda),
             torch.zeros(batch * code_pages, 16, hkv, 128, dtype=torch.int8, device=cuda),
             torch.zeros(batch * code_pages, hkv, dtype=torch.float16, device=cuda),
             torch.zeros(batch * code_pages, hkv, dtype=torch.float16, device=cuda)]
    rq = torch.zeros(batch, hq, 128, dtype=torch.float16, device=cuda)
    q, cos, sin = d(f["query"]), d(f["cos"]), d(f["sin"])
    kc, vc = d(f["key_center"]), d(f["value_center"])
    keys, values = d(f["keys"]), d(f["values"])
    print("golden k2_append", tuple(f["keys"].shape), flush=True)
    for p in range(f["keys"].shape[0]):
        ext.rope_append_page_gauge(q, keys[p], values[p], cos[p], sin[p], kc, vc, rq, *state,
                                   sink, p)
    torch.cuda.synchronize()
    assert_bit_equal(rq, f["expected_rotated_query"], "rotated_query")
    names = ["exact_key_pages", "exact_value_pages", "key_codes", "value_codes", "key_scales",
             "value_scales"]
    for name, got in zip(names, state):
        assert_bit_equal(got, f["expected_" + name], name)


@pytest.mark.parametrize("split", [None, 1])
def test_decode_fixture(cuda, split):
    from pagegauge_amd.decode import PageGaugeSegmentedDecode

    f = load("decode")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    print("golden decode split", split, flush=True)
    dec = PageGaugeSegmentedDecode(torch.empty(8 << 20, dtype=torch.uint8, device=cuda))
    dec.plan(f["indptr"], d(f["indices"]), d(f["last_page_len"]), f["tail_indptr"],
             d(f["tail_indices"]), d(f["tail_last_page_len"]), sm_scale=float(f["sm_scale"]),
             fixed_split_size=split)
    out, lse = dec.run(d(f["query"]), (d(f["k_codes"]), d(f["v_codes"])), d(f["k_scale"]),
                       d(f["v_scale"]), (d(f["tail_k"]), d(f["tail_v"])), d(f["value_center"]),
                       return_lse=True)
    torch.cuda.synchronize()
    assert max_abs(out, f["expected_out_f64"]) <= ATOL_OUT
    assert max_abs(lse, f["expected_lse"]) <= ATOL_LSE


def test_tail_merge_fixture(ext, cuda):
    f = load("tail_merge")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    print("golden tail_merge", tuple(f["query"].shape), flush=True)
    out, lse = d(f["old_output"]), d(f["old_lse"])
    ext.exact_tail_merge_center(d(f["query"]), d(f["exact_key"]), d(f["exact_value"]),
                                d(f["indices"]), d(f["last_page_len"]), out, lse,
                                d(f["value_center"]), float(f["sm_scale"]))
    torch.cuda.synchronize()
    # reference test gates (tests/test_page_gauge_append_extension.py:659-663)
    assert max_abs(out, f["expected_out"]) <= 3e-3
    assert max_abs(lse, f["expected_lse"]) <= ATOL_LSE
