"""Writes the golden fixtures of this directory from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Each ``.npz`` holds inputs and expected outputs (plain arrays, no pickles) of
one small case of the hot path, produced by ``oracle/pg_oracle.py`` whose
functions are pinned by ``tests/test_oracle.py``.  ``tests/test_golden.py``
checks on the CPU that the oracle still reproduces them bit for bit, and
``tests/test_gpu_golden.py`` checks the HIP library against them.

Cases:
  k2_append.npz   fused RoPE + centered append + page finalize, B=2, 2 KV
                  heads, exact sink of 1 page + 2-page tail ring, 3 code
                  pages per request, positions 0..47 (closes 3 pages).
  decode.npz      INT8 page-affine decode + FP16 tail + value center, B=3,
                  8 KV heads (the production shape), ragged (one request
                  without INT8 pages), shuffled pages, partial last pages.
  tail_merge.npz  exact_tail_merge_center, B=2, 2 KV heads, 6-page tails
                  (81 and 96 tokens) through wrapped ring indices.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import pg_oracle as oracle  # noqa: E402

SEED = 20260840


def _f16(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def k2_append(rng):
    batch, sink, tail, code_pages, hkv = 2, 1, 2, 3, 2
    ring = sink + tail
    positions = code_pages * 16
    cos, sin = oracle.rope_tables(positions)
    query = _f16(rng, (batch, 4 * hkv, 128))
    keys = _f16(rng, (positions, batch, hkv, 128))
    values = _f16(rng, (positions, batch, hkv, 128))
    key_center = _f16(rng, (batch, hkv, 128), 0.1)
    value_center = _f16(rng, (batch, hkv, 128), 0.1)
    state = dict(
        rotated_query=np.zeros((batch, 4 * hkv, 128), np.float16),
        exact_key_pages=np.zeros((batch * ring, 16, hkv, 128), np.float16),
        exact_value_pages=np.zeros((batch * ring, 16, hkv, 128), np.float16),
        key_codes=np.zeros((batch * code_pages, 16, hkv, 128), np.int8),
        value_codes=np.zeros((batch * code_pages, 16, hkv, 128), np.int8),
        key_scales=np.zeros((batch * code_pages, hkv), np.float16),
        value_scales=np.zeros((batch * code_pages, hkv), np.float16),
    )
    for p in range(positions):
        oracle.rope_append_page_gauge(query, keys[p], values[p], cos[p], sin[p], key_center,
                                      value_center, exact_sink_pages=sink, position=p, **state)
    return dict(query=query, keys=keys, values=values, cos=cos, sin=sin, key_center=key_center,
                value_center=value_center, exact_sink_pages=np.int32(sink),
                ring_pages=np.int32(ring), code_pages=np.int32(code_pages),
                **{"expected_" + k: v for k, v in state.items()})


def decode(rng):
    pages = 6
    k_codes = rng.integers(-127, 128, (pages, 16, 8, 128)).astype(np.int8)
    v_codes = rng.integers(-127, 128, (pages, 16, 8, 128)).astype(np.int8)
    k_scale = (rng.random((pages, 8)) * 0.02 + 2e-3).astype(np.float16)
    v_scale = (rng.random((pages, 8)) * 0.02 + 2e-3).astype(np.float16)
    indices = rng.permutation(pages).astype(np.int32)
    indptr = np.array([0, 4, 4, 6], np.int32)
    last = np.array([16, 16, 3], np.int32)
    tail_pages = 3
    tail_k = _f16(rng, (tail_pages, 16, 8, 128), 0.4)
    tail_v = _f16(rng, (tail_pages, 16, 8, 128), 0.4)
    tail_indices = rng.permutation(tail_pages).astype(np.int32)
    tail_indptr = np.array([0, 1, 2, 3], np.int32)
    tail_last = np.array([7, 16, 1], np.int32)
    query = _f16(rng, (3, 32, 128))
    value_center = _f16(rng, (3, 8, 128), 0.2)
    sm_scale = np.float32(1.0 / math.sqrt(128))
    out, lse, out64 = oracle.decode(query, k_codes, v_codes, indptr, indices, last,
                                    float(sm_scale), k_scale=k_scale, v_scale=v_scale,
                                    tail_k=tail_k, tail_v=tail_v, tail_indptr=tail_indptr,
                                    tail_indices=tail_indices, tail_last_page_len=tail_last,
                                    value_center=value_center)
    return dict(query=query, k_codes=k_codes, v_codes=v_codes, k_scale=k_scale, v_scale=v_scale,
                indptr=indptr, indices=indices, last_page_len=last, tail_k=tail_k, tail_v=tail_v,
                tail_indptr=tail_indptr, tail_indices=tail_indices, tail_last_page_len=tail_last,
                value_center=value_center, sm_scale=sm_scale, expected_out=out,
                expected_lse=lse, expected_out_f64=out64)


def tail_merge(rng):
    batch, ring, n, hkv = 2, 7, 6, 2
    exact_key = _f16(rng, (batch * ring, 16, hkv, 128), 0.35)
    exact_value = _f16(rng, (batch * ring, 16, hkv, 128), 0.35)
    indices = np.concatenate([r * ring + (np.arange(4, 4 + n) % ring) for r in range(batch)])
    indices = indices.astype(np.int32)
    # a request's tail is (n-1)*16 + last tokens
    last = np.array([1, 16], np.int32)
    tokens_read = [(n - 1) * 16 + int(x) for x in last]
    query = _f16(rng, (batch, 4 * hkv, 128))
    old_output = _f16(rng, (batch, 4 * hkv, 128), 0.2)
    old_lse = (rng.standard_normal((batch, 4 * hkv)) * 0.5 + 8.0).astype(np.float32)
    value_center = _f16(rng, (batch, hkv, 128), 0.1)
    sm_scale = np.float32(1.0 / math.sqrt(128))
    out, lse = oracle.exact_tail_merge_center(query, exact_key, exact_value, indices, last,
                                              old_output, old_lse, value_center, float(sm_scale))
    return dict(query=query, exact_key=exact_key, exact_value=exact_value, indices=indices,
                last_page_len=last, tokens_read=np.array(tokens_read, np.int32),
                old_output=old_output, old_lse=old_lse, value_center=value_center,
                sm_scale=sm_scale, expected_out=out, expected_lse=lse)


CASES = {"k2_append": k2_append, "decode": decode, "tail_merge": tail_merge}


def build(name: str) -> dict:
    return CASES[name](np.random.default_rng(SEED + sorted(CASES).index(name)))


def main() -> None:
    for name in CASES:
        arrays = build(name)
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(name, sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
