"""The C-ABI boundary on the CPU: the library loads, exports every symbol
``include/pagegauge_hip.h`` declares (and nothing else), the ctypes
prototypes agree with the header, and the host-only entry points validate as
documented; likewise bench.py's probe library against
``include/pagegauge_bench.h``.  No GPU compute is called here."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

from pagegauge_amd import _capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pagegauge_hip.h"
BENCH_HEADER = ROOT / "include" / "pagegauge_bench.h"


def _declarations(header=HEADER) -> dict[str, int]:
    """name -> parameter count of every function declared in the header."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    out = {}
    for match in re.finditer(r"^(?:const\s+)?[a-z_0-9]+\s*\*?\s*(pg_[a-z_0-9]+)\s*\(([^;]*?)\)\s*;",
                             text, flags=re.M | re.S):
        params = match.group(2).strip()
        out[match.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_header_declares_the_expected_entry_points():
    names = set(_declarations())
    assert {"pg_rope_append_fp16", "pg_rope_append_page_gauge", "pg_decode_plan",
            "pg_decode_run", "pg_exact_tail_merge_center", "pg_merge_state_in_place"} <= names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_capi.LIBRARY_PATH))
    for name in _declarations():
        assert hasattr(lib, name), name
    exported = subprocess.run(["nm", "-D", "--defined-only", str(_capi.LIBRARY_PATH)],
                              capture_output=True, text=True, check=True).stdout
    public = set(re.findall(r" T (pg_[a-z_0-9]+)$", exported, flags=re.M))
    assert public == set(_declarations()), "exports and header disagree"


def test_ctypes_prototypes_match_header_arity():
    declared = _declarations()
    assert set(_capi.PROTOTYPES) == set(declared)
    for name, (_, argtypes) in _capi.PROTOTYPES.items():
        assert len(argtypes) == declared[name], name


def test_bench_library_exports_its_header_and_nothing_of_the_product():
    """The probes live in libpagegauge_bench.so; the product exports none of
    them.  pg_trace_set_buffer is declared there too but exported only by the
    trace build of the product library."""
    declared = _declarations(BENCH_HEADER)
    assert {"pg_probe_linear_read", "pg_probe_page_walk", "pg_probe_decode_walk"} <= set(declared)
    exported = subprocess.run(["nm", "-D", "--defined-only", str(_capi.BENCH_LIBRARY_PATH)],
                              capture_output=True, text=True, check=True).stdout
    public = set(re.findall(r" T (pg_[a-z_0-9]+)$", exported, flags=re.M))
    assert public == set(declared) - {"pg_trace_set_buffer"}
    for name, (_, argtypes) in {**_capi.BENCH_PROTOTYPES, **_capi.TRACE_PROTOTYPES}.items():
        assert len(argtypes) == declared[name], name
    assert not any(name.startswith("pg_probe") for name in _declarations())
    assert _capi.bench_library().pg_abi_version() == _capi.ABI_VERSION


def test_library_loads_and_reports_abi_version():
    lib = _capi.library()
    assert lib.pg_abi_version() == _capi.ABI_VERSION


def test_plan_struct_layout_matches_header():
    text = HEADER.read_text()
    body = re.search(r"typedef struct pg_decode_plan \{(.*?)\} pg_decode_plan_t;", text, re.S).group(1)
    fields = re.findall(r"(int32_t|int64_t)\s+([a-z_0-9]+);", body)
    assert [n for _, n in fields] == [n for n, _ in _capi.DecodePlan._fields_]
    sizes = {"int32_t": 4, "int64_t": 8}
    for (ctype, name), (_, ftype) in zip(fields, _capi.DecodePlan._fields_):
        assert ctypes.sizeof(ftype) == sizes[ctype], name


def test_workspace_bytes_closed_form():
    lib = _capi.library()
    # items (48 B each) + item_ptr + partials (B * Hq * items * (128 + 2) floats), 256-aligned
    got = lib.pg_decode_workspace_bytes(1, 32, 193, 193)
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert got == align(193 * 48) + align(2 * 4) + align(32 * 193 * 130 * 4)
    assert lib.pg_decode_workspace_bytes(0, 32, 1, 1) == 0


def test_select_split_pages_is_the_balanced_planners_choice():
    from pagegauge_amd import decode

    lib = _capi.library()
    for pages, batch, nbytes, cus in ((3072, 1, 4096, 256), (100, 1, 4096, 256),
                                      (8192, 8, 4096, 256), (8195, 8, 4096, 256),
                                      (3072, 1, 8192, 256), (20480, 4, 4096, 128)):
        per, extra = divmod(pages, batch)
        indptr = [0]
        for b in range(batch):
            indptr.append(indptr[-1] + per + (b < extra))
        plan, _, _ = decode.plan_work_items(
            torch.tensor(indptr, dtype=torch.int32), torch.full((batch,), 16, dtype=torch.int32),
            kv_data_type=torch.int8 if nbytes == 4096 else torch.float16, num_cus=cus)
        assert lib.pg_select_split_pages(pages, batch, 8, nbytes, cus) == plan.split_pages
    assert lib.pg_select_split_pages(3072, 1, 8, 4096, 256) == 28     # the B1/49K medium plan
    # more pages than 4096 items of 64 pages: no plan
    assert lib.pg_select_split_pages(10 ** 6, 1, 8, 4096, 256) == 0
    assert "too many splits" in _capi.last_error()
    assert lib.pg_select_split_pages(3072, 1, 8, 1000, 256) == 0
    assert "bytes_per_page" in _capi.last_error()


@pytest.mark.parametrize("kwargs,code,message", [
    (dict(head_dim=64), 3, "head dimension must be 128"),
    (dict(page_size=32), 3, "page size must be 16"),
    (dict(num_qo_heads=16), 3, "GQA group size 4"),
    (dict(last=[17]), 1, r"last_page_len must lie in \[1, 16\]"),
])
def test_host_plan_validation_messages(kwargs, code, message):
    from pagegauge_amd.decode import plan_work_items

    args = dict(indptr=[0, 40], last=[16], num_qo_heads=32, head_dim=128, page_size=16)
    args.update(kwargs)
    with pytest.raises(RuntimeError, match=message) as info:
        plan_work_items(args["indptr"], args["last"], num_qo_heads=args["num_qo_heads"],
                        head_dim=args["head_dim"], page_size=args["page_size"])
    assert f"(code {code})" in str(info.value)


def test_c_planner_rejects_a_decreasing_indptr():
    """The Python wrappers reject it first; the C planner checks it too."""
    import ctypes

    import torch

    lib = _capi.library()
    indptr = torch.tensor([5, 3], dtype=torch.int32)
    last = torch.tensor([16], dtype=torch.int32)
    plan = _capi.DecodePlan()
    rc = lib.pg_decode_plan_host(indptr.data_ptr(), last.data_ptr(), 1, _capi.PG_KV_INT8, None,
                                 None, 32, 8, 128, 16, 0, 0, 0, 256, ctypes.byref(plan), None, 0,
                                 None)
    assert rc == 1 and "indptr must be non-decreasing" in _capi.last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_capi, "_library", None)
    monkeypatch.setattr(_capi, "LIBRARY_PATH", tmp_path / "absent.so")
    with pytest.raises(_capi.LibraryMissingError, match="missing"):
        _capi.library()
