"""The committed golden fixtures (``tests/golden/*.npz``) on the CPU: the
oracle regenerates them bit for bit, and the C restatement agrees with the
decode fixture."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import pytest

from oracle import c_oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


@pytest.mark.parametrize("name", ["k2_append", "decode", "tail_merge"])
def test_oracle_reproduces_fixture(name):
    fixture = load(name)
    regenerated = _maker().build(name)
    assert set(fixture) == set(regenerated)
    for key, value in regenerated.items():
        want = fixture[key]
        assert want.dtype == value.dtype and want.shape == value.shape, key
        assert np.array_equal(np.ascontiguousarray(want).view(np.uint8),
                              np.ascontiguousarray(value).view(np.uint8)), key


def test_c_oracle_matches_decode_fixture():
    f = load("decode")
    out, lse = c_oracle.decode_page_gauge(
        f["query"], f["k_codes"], f["v_codes"], f["k_scale"], f["v_scale"], f["indptr"],
        f["indices"], f["last_page_len"], float(f["sm_scale"]), f["tail_k"], f["tail_v"],
        f["tail_indptr"], f["tail_indices"], f["tail_last_page_len"], f["value_center"])
    assert np.abs(out.astype(np.float64) - f["expected_out_f64"]).max() < 2e-3
    np.testing.assert_allclose(lse, f["expected_lse"], atol=1e-4)


def test_fixture_cases_hit_the_edge_cases():
    d = load("decode")
    counts = np.diff(d["indptr"])
    assert (counts == 0).any() and (d["last_page_len"] < 16).any()
    assert (d["tail_last_page_len"] == 1).any()
    k2 = load("k2_append")
    assert k2["expected_key_scales"].all()              # every code page closed
    t = load("tail_merge")
    assert list(t["tokens_read"]) == [81, 96]
