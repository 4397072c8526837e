"""Shared helpers of the test suite (CPU copies, oracle calls)."""

from __future__ import annotations

import numpy as np

from oracle import pg_oracle as oracle


def cpu(tensor) -> np.ndarray:
    return tensor.detach().cpu().numpy()


def bits(array: np.ndarray) -> np.ndarray:
    """Byte view for bit-exact comparisons (NaN payloads and -0 included)."""
    return np.ascontiguousarray(array).view(np.uint8)


def assert_bit_equal(got, want, what: str = "") -> None:
    got = cpu(got) if not isinstance(got, np.ndarray) else got
    if got.shape != want.shape or not np.array_equal(bits(got), bits(want)):
        diff = np.flatnonzero(bits(got).ravel() != bits(want).ravel())
        raise AssertionError(f"{what}: {diff.size} differing bytes (first at {diff[:5]})")


def oracle_decode(w, with_tail: bool = True, with_center: bool = True):
    """Oracle (float64) decode of a ``pagegauge_amd.workloads.DecodeWorkload``."""
    kw = {}
    if with_tail:
        kw.update(tail_k=cpu(w.tail_k), tail_v=cpu(w.tail_v), tail_indptr=cpu(w.tail_indptr),
                  tail_indices=cpu(w.tail_indices), tail_last_page_len=cpu(w.tail_last_page_len))
    if with_center:
        kw["value_center"] = cpu(w.value_center)
    return oracle.decode(cpu(w.query), cpu(w.k_codes), cpu(w.v_codes), cpu(w.old_indptr),
                         cpu(w.old_indices), cpu(w.old_last_page_len), w.sm_scale,
                         k_scale=cpu(w.k_scale), v_scale=cpu(w.v_scale), **kw)


def max_abs(a, b) -> float:
    a = cpu(a) if not isinstance(a, np.ndarray) else a
    b = cpu(b) if not isinstance(b, np.ndarray) else b
    return float(np.abs(a.astype(np.float64) - b.astype(np.float64)).max())
