"""Host-side argument checks of the C ABI, run without a GPU.

Every case below fails a check that the entry point makes before it touches
the HIP runtime, so the call returns an error code and a message and launches
nothing.  The messages of the cache-update checks are the ones the
reference's tests assert ("must be nonnegative", "at least one tail-ring
page", "logical cache capacity": tests/test_page_gauge_append_extension.py
:520-585).  Cases pass stand-in (non-null, never dereferenced) pointers to
get past the null checks, so the module is skipped wherever a GPU is
visible: a check that regressed there must not turn into a launch on such an
address.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from pagegauge_amd import _capi

pytestmark = pytest.mark.skipif(torch.cuda.is_available(),
                                reason="host-only checks: stand-in pointers are never launched")

FAKE = 0x1000          # stand-in device address (a failing check returns before any use)


def _call(name, *args):
    rc = getattr(_capi.library(), name)(*args)
    return rc, _capi.last_error()


def _rope_append_page_gauge(**over):
    a = dict(query=FAKE, key=FAKE, value=FAKE, cosine=FAKE, sine=FAKE, key_center=FAKE,
             value_center=FAKE, center_batch_stride=8 * 128, rotated_query=FAKE,
             exact_key=FAKE, exact_value=FAKE, key_codes=FAKE, value_codes=FAKE,
             key_scales=FAKE, value_scales=FAKE, qbs=32 * 128, kbs=8 * 128, vbs=8 * 128,
             batch=1, qh=32, kvh=8, exact_pages=16, sink=0, code_pages=64, position=100,
             device_position=None, rope_row_stride=128, rope_rows=0, stream=None)
    a.update(over)
    return _call("pg_rope_append_page_gauge", *a.values())


@pytest.mark.parametrize("over,code,message", [
    (dict(batch=0), 1, "batch sizes must match and be positive"),
    (dict(kvh=0), 1, "head counts must be positive"),
    (dict(key_codes=None), 1, "null tensor pointer"),
    (dict(sink=-1), 1, "must be nonnegative"),
    (dict(exact_pages=2, sink=2), 1, "at least one tail-ring page"),
    (dict(exact_pages=20, sink=5, code_pages=5), 1, "logical cache capacity"),
    (dict(position=-1), 1, "position must be non-negative"),
    (dict(position=64 * 16), 1, "exceeds the per-request PageGauge cache capacity"),
    (dict(device_position=FAKE, rope_rows=0), 1, "dynamic RoPE tables"),
])
def test_rope_append_page_gauge_rejects(over, code, message):
    rc, text = _rope_append_page_gauge(**over)
    assert rc == code
    assert message in text


def _gemv(**over):
    a = dict(weight=FAKE, n=4096, k=4096, x=FAKE, x_stride=4096, batch=1, norm=None,
             eps=ctypes.c_float(1e-5), swiglu=0, residual=None, residual_stride=0, out=FAKE,
             out_stride=4096, out_f32=0, stream=None)
    a.update(over)
    return _call("pg_decoder_gemv", *a.values())


@pytest.mark.parametrize("over,code,message", [
    (dict(weight=None), 1, "null tensor pointer"),
    (dict(k=4000), 1, "multiple of 512"),
    (dict(batch=5), 3, "batch of 1 to 4 rows"),
    (dict(swiglu=1, n=4095), 1, "even n"),
    (dict(x_stride=4100), 1, "row strides must cover the rows"),
    (dict(out_stride=100), 1, "row strides must cover the rows"),
])
def test_decoder_gemv_rejects(over, code, message):
    rc, text = _gemv(**over)
    assert rc == code
    assert message in text


@pytest.mark.parametrize("args,message", [
    ((None, 1, 10, 10, FAKE, None), "null tensor pointer"),
    ((FAKE, 1, 0, 10, FAKE, None), "at least one element"),
])
def test_argmax_rejects(args, message):
    rc, text = _call("pg_argmax_f32", *args)
    assert rc == 1
    assert message in text


def test_decode_run_rejects_a_null_plan():
    args = [None] * len(_capi.PROTOTYPES["pg_decode_run"][1])
    args[17] = ctypes.c_float(0.088)         # sm_scale
    args[2] = 0
    args[14] = 0
    rc, text = _call("pg_decode_run", *args)
    assert rc == 1
    assert "null run argument" in text


def test_errors_do_not_leak_into_the_next_call():
    rc, text = _gemv(weight=None)
    assert rc == 1 and text
    rc, text = _call("pg_argmax_f32", FAKE, 1, 0, 10, FAKE, None)
    assert "at least one element" in text and "null" not in text


def _host_plan(kind=_capi.PG_KV_INT8, tail=True):
    """A real plan from the host planner (one request of 100 INT8 pages and a
    16-page FP16 tail)."""
    from pagegauge_amd.decode import plan_work_items

    dtype = {_capi.PG_KV_INT8: torch.int8, _capi.PG_KV_HETEROGENEOUS: "heterogeneous"}[kind]
    plan, _, _ = plan_work_items([0, 100], [16], [0, 16] if tail else None,
                                 [16] if tail else None, kv_data_type=dtype)
    return plan


def _decode_run(plan, **over):
    a = dict(plan=ctypes.byref(plan), q=FAKE, qbs=4096, k=FAKE, v=FAKE, ks=FAKE, vs=FAKE, idx=FAKE,
             last=FAKE, tk=FAKE, tv=FAKE, tidx=FAKE, tlast=FAKE, center=FAKE, cbs=1024, out=FAKE,
             lse=FAKE, scale=ctypes.c_float(0.088), ws=FAKE, stream=None)
    a.update(over)
    return _call("pg_decode_run", *a.values())


@pytest.mark.parametrize("over,message", [
    (dict(q=None), "null run argument"),
    (dict(ws=None), "null run argument"),
    (dict(k=None), "primary segment tensors missing"),
    (dict(ks=None), "INT8 pages need k_scale and v_scale"),
    (dict(tidx=None), "tail segment tensors missing"),
    (dict(scale=ctypes.c_float(0.0)), "sm_scale must be positive and finite"),
    (dict(scale=ctypes.c_float(float("inf"))), "sm_scale must be positive and finite"),
])
def test_decode_run_rejects(over, message):
    rc, text = _decode_run(_host_plan(), **over)
    assert rc == 1
    assert message in text


def test_decode_run_rejects_a_tampered_plan():
    plan = _host_plan()
    plan.waves_per_block = 3
    rc, text = _decode_run(plan)
    assert rc == 1 and "invalid waves_per_block" in text
    plan = _host_plan()
    assert plan.closed_form == 1
    plan.cf_tail_items = plan.num_items + 1
    rc, text = _decode_run(plan)
    assert rc == 1 and "inconsistent closed-form" in text


def test_heterogeneous_plans_and_old_kv_len_go_together():
    # an INT8 plan given old_kv_len (the heterogeneous entry point)
    # plan, q, q stride, codes k/v, scales k/v, exact k/v, indices, last_page_len, old_kv_len,
    # value_center, center stride, out, lse, sm_scale, workspace, stream
    args = [ctypes.byref(_host_plan()), FAKE, 4096, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
            FAKE, FAKE, 1024, FAKE, FAKE, ctypes.c_float(0.088), FAKE, None]
    rc, text = _call("pg_decode_run_heterogeneous", *args)
    assert rc == 1 and "old_kv_len goes with (and only with) a heterogeneous plan" in text
    # a heterogeneous plan without the exact pages
    args[0] = ctypes.byref(_host_plan(_capi.PG_KV_HETEROGENEOUS, tail=False))
    args[7] = None                       # exact_k
    rc, text = _call("pg_decode_run_heterogeneous", *args)
    assert rc == 1 and "heterogeneous pages need the exact K/V pages" in text


def test_finalize_needs_int8_pages_and_positive_code_pages():
    args = [ctypes.byref(_host_plan()), FAKE, 4096, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
            FAKE, FAKE, FAKE, 1024, FAKE, FAKE, ctypes.c_float(0.088), FAKE, FAKE, 0, 0, None]
    rc, text = _call("pg_decode_run_finalize", *args)
    assert rc == 1 and "positive code pages per request" in text


# --- host page tables checked before the planner reads them ----------------

@pytest.mark.parametrize("indptr,last,message", [
    ([0, 3, 5, 9], [16], "last_page_len must have one entry per request (3), got 1"),
    ([0, 3, 5, 9], [16, 16, 16, 16], "one entry per request"),
    ([-2, 3], [16], "indptr[0] must be non-negative"),
    ([0, 5, 3], [16, 16], "indptr must be non-decreasing"),
    ([0], [], "batch_size + 1 >= 2 entries"),
])
def test_plan_rejects_inconsistent_tables(indptr, last, message):
    from pagegauge_amd import decode

    with pytest.raises(ValueError, match=message.replace("(", r"\(").replace(")", r"\)")
                       .replace("[", r"\[").replace("]", r"\]").replace("+", r"\+")):
        decode.plan_work_items(indptr, last)


def test_plan_rejects_a_short_tail_table():
    from pagegauge_amd import decode

    with pytest.raises(ValueError, match="tail last_page_len must have one entry per request"):
        decode.plan_work_items([0, 3, 5], [16, 16], tail_indptr=[0, 1, 2], tail_last_page_len=[16])
    with pytest.raises(ValueError, match="cover the same batch"):
        decode.plan_work_items([0, 3, 5], [16, 16], tail_indptr=[0, 1], tail_last_page_len=[16])
    with pytest.raises(ValueError, match="go together"):
        decode.plan_work_items([0, 3], [16], tail_indptr=[0, 1])


def test_host_tables_checks_the_indices_length():
    from pagegauge_amd import decode

    indices = torch.arange(8, dtype=torch.int32)
    decode._host_tables([0, 3, 8], [16, 16], indices)           # exactly long enough
    with pytest.raises(ValueError, match="indices has 8 entries but indptr\\[-1\\] is 9"):
        decode._host_tables([0, 3, 9], [16, 16], indices)


def test_page_id_check_is_opt_in(monkeypatch):
    from pagegauge_amd import decode

    ids = torch.tensor([4, 0, 7, 2], dtype=torch.int32)
    indptr = torch.tensor([1, 3], dtype=torch.int32)          # planned ids: 0, 7
    monkeypatch.setattr(decode, "CHECK_PAGE_IDS", False)
    assert decode._page_id_range(ids, indptr) is None
    monkeypatch.setattr(decode, "CHECK_PAGE_IDS", True)
    span = decode._page_id_range(ids, indptr)
    assert span == (0, 7)
    decode._check_page_ids(span, 8, "INT8")
    with pytest.raises(ValueError, match=r"INT8 page ids span \[0, 7\] but the pool holds 7 pages"):
        decode._check_page_ids(span, 7, "INT8")
    with pytest.raises(ValueError, match="span \\[-1, 3\\]"):
        decode._check_page_ids((-1, 3), 8, "exact")


@pytest.mark.parametrize("args,message", [
    ((0, 16, 16, 4, 4, 1, 0), "null tensor pointer"),
    ((16, 16, 6, 4, 2, 1, 0), "whole items"),          # pages_per_item not a multiple of 4
    ((16, 18, 8, 4, 2, 1, 0), "whole items"),          # pages not whole items
    ((16, 16, 16, 2, 2, 1, 0), "heads_per_block"),
    ((16, 16, 16, 8, 3, 1, 0), "depth"),
    ((16, 16, 16, 4, 2, 2, 0), "mode"),                # whole pages need 8 heads per block
    ((16, 64, 4, 4, 2, 0, 0), "an entry per workgroup"),  # 16 workgroups, a 15-entry sink
])
def test_decode_walk_probe_rejects(args, message):
    """Argument checks of pg_probe_decode_walk run before any launch (no GPU
    needed); fake non-null pointers never reach a kernel."""
    lib = _capi.bench_library()
    ptr, pages, per_item, heads, depth, mode, _ = args
    fake = ptr or None
    rc = lib.pg_probe_decode_walk(fake, fake, fake, pages, per_item, heads, depth, mode, fake,
                                  15, None, None, None)
    assert rc == 1 and message in lib.pg_last_error().decode()


def test_read_probes_reject_a_short_sink():
    lib = _capi.bench_library()
    fake = 16
    assert lib.pg_probe_linear_read(fake, 1 << 20, fake, 511, 512, None, None, None) == 1
    assert "an entry per workgroup (512 > 511)" in lib.pg_last_error().decode()
    assert lib.pg_probe_page_walk(fake, fake, fake, 40, 4, 16384, fake, 9, None, None, None) == 1
    assert "(10 > 9)" in lib.pg_last_error().decode()
