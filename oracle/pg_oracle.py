"""CPU oracle for the PageGauge compressed-KV decode path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
use it, and only as the checker.

Every function restates one reference function and cites the file:line it
follows (paths relative to the PageGauge reference tree).  Precision rules:

* An FP16 operation of the reference (``mul.rn.f16``/``add.rn.f16``) is
  evaluated exactly in float64 and rounded once to float16 (numpy's
  float64->float16 conversion is IEEE round-to-nearest-even, subnormals kept).
  The exact product of two halves needs 22 significant bits and the exact sum
  at most 51, so one rounding from float64 equals the correctly rounded FP16
  result.
* An FP32 operation of the reference is evaluated in numpy float32, which is
  IEEE round-to-nearest-even (division included).
* Attention outputs are computed in float64 (dense softmax over the
  dequantised cache) and rounded to float16 at the end.

Pinning status of each function (how a plausible mistake is caught) is listed
in ``PINNED``; every function is pinned by at least one check in
``tests/test_oracle.py`` against the reference's own golden lists, the
reference tests' torch formulas run on the CPU, closed forms, or brute force.
"""

from __future__ import annotations

from typing import Optional

import numpy as np

PAGE = 16
DIM = 128
HALF_DIM = DIM // 2
LOG2E = 1.4426950408889634
SCALE_FLOOR = np.float32(2.0 ** -20)

PINNED = {
    "rope_rotate": "torch fp16 formula of tests/test_page_gauge_append_extension.py:77-84",
    "rope_append_fp16": "identity RoPE + request-major placement, "
    "tests/test_page_gauge_append_extension.py:766-786",
    "rope_append_page_gauge": "torch formulas for centering and scale, "
    "tests/test_page_gauge_overheads.py:54-63; ring/code placement golden cases",
    "finalize_codes": "brute-force exact-rational evaluation of floor(rn32(q+0.5))",
    "quantize_page_gauge": "torch transcription of scripts/benchmark_flashinfer_page_affine_int8.py:256-278",
    "quantize_completed_kv_pages": "torch transcription of scripts/benchmark_page_gauge_overheads.py:23-83",
    "append_finalize_page_gauge": "equivalence with rope_append_page_gauge at identity RoPE",
    "append_kv": "the reference's cross-check of its two appends "
    "(scripts/benchmark_page_gauge_overheads.py:556-609: fused exact pages + center within "
    "2e-3 of the plain pages, codes reconstruct them < 0.03) and direct placement",
    "rope_append_page_gauge_slots": "equivalence with rope_append_page_gauge_positions when the "
    "ids are the request-major slots (tests/test_oracle.py, CPU), skipped rows for bad ids",
    "decode": "torch float64 softmax attention; logsumexp identity; merge associativity",
    "merge_state": "decode(A u B) == merge(decode(A), decode(B))",
    "exact_tail_merge_center": "torch oracle of tests/test_page_gauge_append_extension.py:628-657",
    "exact_center": "exact-rational (Fraction) mean rounded f64 -> f32 -> f16",
    "decode_heterogeneous": "dense float64 softmax over the logical sequence (old pages "
    "reconstructed, then exact pages) of diagnostics/benchmark_heterogeneous_fa2_correctness.py:"
    "291-299 on its nine boundary CASES (:63-73)",
}


# ---------------------------------------------------------------------------
# scalar helpers
# ---------------------------------------------------------------------------

def f16(x) -> np.ndarray:
    """Round (exactly given) values once to IEEE binary16, RN-even."""
    return np.asarray(x, dtype=np.float64).astype(np.float16)


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def _as_f16(array) -> np.ndarray:
    array = np.asarray(array)
    if array.dtype != np.float16:
        raise TypeError(f"expected float16 array, got {array.dtype}")
    return array


# ---------------------------------------------------------------------------
# A1: RoPE (tests/page_gauge_append_extension.cu:148-180)
# ---------------------------------------------------------------------------

def rope_rotate(x: np.ndarray, cosine: np.ndarray, sine: np.ndarray) -> np.ndarray:
    """HF-exact FP16 RoPE over the last (128) axis.

    Follows ``rotate_element`` (tests/page_gauge_append_extension.cu:148-180):
    partner = x[d+64] with its sign bit flipped for d<64, x[d-64] for d>=64;
    y = rn16(rn16(x*cos) + rn16(partner*sin)), each operation rounded
    separately (no FMA).  ``cosine``/``sine`` broadcast over leading axes.
    """
    x = _as_f16(x)
    cosine = _as_f16(cosine)
    sine = _as_f16(sine)
    partner = np.concatenate((-x[..., HALF_DIM:], x[..., :HALF_DIM]), axis=-1)
    primary = f16(x.astype(np.float64) * cosine.astype(np.float64))
    secondary = f16(partner.astype(np.float64) * sine.astype(np.float64))
    return f16(primary.astype(np.float64) + secondary.astype(np.float64))


# ---------------------------------------------------------------------------
# A3: completed-page finalize (tests/page_gauge_append_extension.cu:327-382)
# ---------------------------------------------------------------------------

def page_scale(values_f32: np.ndarray, axis) -> np.ndarray:
    """fp16(max(amax|v| / 127, 2^-20)) with an IEEE float32 division.

    tests/page_gauge_append_extension.cu:343-348 (block_max starts at 0).
    """
    amax = np.abs(f32(values_f32)).max(axis=axis, initial=np.float32(0.0))
    amax = f32(amax)
    quotient = f32(amax / np.float32(127.0))
    return np.maximum(quotient, SCALE_FLOOR).astype(np.float16)


def sign_symmetric_round(quotient_f32: np.ndarray) -> np.ndarray:
    """q>=0 ? floor(rn32(q+0.5)) : -floor(rn32(-q+0.5)), clamped to [-127,127].

    tests/page_gauge_append_extension.cu:371-378 and
    scripts/benchmark_page_gauge_overheads.py:64-73.  The float32 addition can
    round up (q = 0.5 - 2^-25 gives 1); that quirk is reproduced.
    """
    q = f32(quotient_f32)
    positive = np.floor(f32(q + np.float32(0.5)))
    negative = -np.floor(f32(-q + np.float32(0.5)))
    rounded = np.where(q >= np.float32(0.0), positive, negative)
    return np.clip(rounded, -127, 127).astype(np.int8)


def finalize_codes(page_f16: np.ndarray, axis) -> tuple[np.ndarray, np.ndarray]:
    """Return (codes int8, scale fp16) of one completed page/head block.

    Reads the FP16-stored centered values as float32, as the reference kernel
    reloads them (tests/page_gauge_append_extension.cu:333-382).
    """
    values = _as_f16(page_f16).astype(np.float32)
    scale = page_scale(values, axis=axis)
    scale_f32 = np.expand_dims(scale.astype(np.float32), axis)
    codes = sign_symmetric_round(f32(values / scale_f32))
    return codes, scale


# ---------------------------------------------------------------------------
# K2: fused append kernels (tests/page_gauge_append_extension.cu:182-383)
# ---------------------------------------------------------------------------

def _position_valid(position: int, capacity_tokens: int, rope_rows: Optional[int]) -> bool:
    if position < 0 or position >= capacity_tokens:
        return False
    if rope_rows is not None and position >= rope_rows:
        return False
    return True


def rope_append_fp16(query, key, value, cosine, sine, rotated_query, key_pages,
                     value_pages, position: int, rope_rows: Optional[int] = None) -> None:
    """In-place restatement of ``rope_append_fp16_kernel``.

    tests/page_gauge_append_extension.cu:182-242: every request writes its
    rotated key and raw value at physical page ``request*P + position//16``.
    ``cosine``/``sine`` are the [128] rows for ``position``.  Out-of-range
    positions are silent no-ops (``:203-207``).
    """
    batch = query.shape[0]
    pages_per_request = key_pages.shape[0] // batch
    if not _position_valid(position, pages_per_request * PAGE, rope_rows):
        return
    page, token = divmod(position, PAGE)
    rotated_query[...] = rope_rotate(query, cosine, sine)
    rotated_key = rope_rotate(key, cosine, sine)
    for request in range(batch):
        physical = request * pages_per_request + page
        key_pages[physical, token] = rotated_key[request]
        value_pages[physical, token] = value[request]


def _center_for(center: np.ndarray, request: int) -> np.ndarray:
    # [B,Hkv,128] or [Hkv,128] for batch one (:730-739)
    return center if center.ndim == 2 else center[request]


def _append_centered_and_finalize(request_key_rot, request_value, key_center, value_center,
                                  exact_key_pages, exact_value_pages, key_codes, value_codes,
                                  key_scales, value_scales, exact_page: int, code_page: int,
                                  token: int) -> None:
    centered_key = f16(f32(request_key_rot) - f32(key_center))
    centered_value = f16(f32(request_value) - f32(value_center))
    exact_key_pages[exact_page, token] = centered_key
    exact_value_pages[exact_page, token] = centered_value
    if token != PAGE - 1:
        return
    # ring page [16, Hkv, 128]; reduction over tokens and dims per head
    codes_k, scale_k = finalize_codes(exact_key_pages[exact_page], axis=(0, 2))
    codes_v, scale_v = finalize_codes(exact_value_pages[exact_page], axis=(0, 2))
    key_codes[code_page] = codes_k
    value_codes[code_page] = codes_v
    key_scales[code_page] = scale_k
    value_scales[code_page] = scale_v


def rope_append_page_gauge(query, key, value, cosine, sine, key_center, value_center,
                           rotated_query, exact_key_pages, exact_value_pages, key_codes,
                           value_codes, key_scales, value_scales, exact_sink_pages: int,
                           position: int, rope_rows: Optional[int] = None) -> None:
    """In-place restatement of ``rope_append_page_gauge_kernel``.

    tests/page_gauge_append_extension.cu:244-383: ring slot
    ``req*E + (page < S ? page : S + page % (E-S))`` (:288-293), centered FP16
    K/V write (:316-325), and on the page's last token the INT8 finalize into
    code page ``req*Pc + page`` (:327-382).
    """
    batch = query.shape[0]
    exact_pages_per_request = exact_key_pages.shape[0] // batch
    code_pages_per_request = key_codes.shape[0] // batch
    if not _position_valid(position, code_pages_per_request * PAGE, rope_rows):
        return
    page, token = divmod(position, PAGE)
    tail_pages = exact_pages_per_request - exact_sink_pages
    local = page if page < exact_sink_pages else exact_sink_pages + page % tail_pages
    rotated_query[...] = rope_rotate(query, cosine, sine)
    rotated_key = rope_rotate(key, cosine, sine)
    for request in range(batch):
        _append_centered_and_finalize(
            rotated_key[request], value[request],
            _center_for(key_center, request), _center_for(value_center, request),
            exact_key_pages, exact_value_pages, key_codes, value_codes,
            key_scales, value_scales,
            request * exact_pages_per_request + local,
            request * code_pages_per_request + page, token)


def rope_append_page_gauge_positions(query, key, value, cosine_table, sine_table, positions,
                                     key_center, value_center, rotated_query, exact_key_pages,
                                     exact_value_pages, key_codes, value_codes, key_scales,
                                     value_scales, exact_sink_pages: int) -> None:
    """Per-request-position variant: the scalar kernel applied row by row.

    Each request ``r`` behaves exactly as ``rope_append_page_gauge`` with
    ``position = positions[r]`` and the RoPE row ``cosine_table[positions[r]]``
    (the per-request semantics of scripts/benchmark_page_gauge_overheads.py:112-205,
    with the RoPE and ring/code index spaces of the CUDA kernel).
    """
    batch = query.shape[0]
    exact_pages_per_request = exact_key_pages.shape[0] // batch
    code_pages_per_request = key_codes.shape[0] // batch
    rope_rows = cosine_table.shape[0]
    tail_pages = exact_pages_per_request - exact_sink_pages
    for request in range(batch):
        position = int(positions[request])
        if not _position_valid(position, code_pages_per_request * PAGE, rope_rows):
            continue
        page, token = divmod(position, PAGE)
        local = page if page < exact_sink_pages else exact_sink_pages + page % tail_pages
        cosine = cosine_table[position]
        sine = sine_table[position]
        rotated_query[request] = rope_rotate(query[request], cosine, sine)
        rotated_key = rope_rotate(key[request], cosine, sine)
        _append_centered_and_finalize(
            rotated_key, value[request],
            _center_for(key_center, request), _center_for(value_center, request),
            exact_key_pages, exact_value_pages, key_codes, value_codes,
            key_scales, value_scales,
            request * exact_pages_per_request + local,
            request * code_pages_per_request + page, token)


def rope_append_page_gauge_slots(query, key, value, cosine_table, sine_table, positions,
                                 exact_page_ids, code_page_ids, key_center, value_center,
                                 rotated_query, exact_key_pages, exact_value_pages, key_codes,
                                 value_codes, key_scales, value_scales) -> None:
    """Serving-table variant: row ``r`` appends at ``positions[r]`` into exact
    page ``exact_page_ids[r]`` and finalizes into code page ``code_page_ids[r]``
    (the ids of the serving block tables,
    experiments/mlsys2027/serving_v1/pagegauge_vllm/decode_metadata.py:50-60);
    the arithmetic is ``rope_append_page_gauge``'s.  Negative or out-of-pool
    ids skip the row."""
    rope_rows = cosine_table.shape[0]
    for request in range(query.shape[0]):
        position = int(positions[request])
        exact_page, code_page = int(exact_page_ids[request]), int(code_page_ids[request])
        if not (0 <= position < rope_rows and 0 <= exact_page < exact_key_pages.shape[0]
                and 0 <= code_page < key_codes.shape[0]):
            continue
        cosine, sine = cosine_table[position], sine_table[position]
        rotated_query[request] = rope_rotate(query[request], cosine, sine)
        rotated_key = rope_rotate(key[request], cosine, sine)
        _append_centered_and_finalize(
            rotated_key, value[request],
            _center_for(key_center, request), _center_for(value_center, request),
            exact_key_pages, exact_value_pages, key_codes, value_codes,
            key_scales, value_scales, exact_page, code_page, position % PAGE)


def append_kv(key, value, key_pages, value_pages, page_ids, page_offsets) -> None:
    """scripts/benchmark_page_gauge_overheads.py:86-109 (plain FP16 append)."""
    for request in range(key.shape[0]):
        page, token = int(page_ids[request]), int(page_offsets[request])
        key_pages[page, token] = key[request]
        value_pages[page, token] = value[request]


def append_finalize_page_gauge(key, value, key_center, value_center, exact_key_pages,
                               exact_value_pages, key_codes, value_codes, key_scales,
                               value_scales, page_ids, page_offsets) -> None:
    """scripts/benchmark_page_gauge_overheads.py:112-205.

    Centered append at per-request (page, offset) without RoPE; on offset 15 the
    FP16-stored page is reloaded and quantised into the same page index.  The
    centers are shared [H,128] tensors.
    """
    for request in range(key.shape[0]):
        page, token = int(page_ids[request]), int(page_offsets[request])
        _append_centered_and_finalize(
            key[request], value[request], key_center, value_center,
            exact_key_pages, exact_value_pages, key_codes, value_codes,
            key_scales, value_scales, page, page, token)


# ---------------------------------------------------------------------------
# Bulk quantizers (cache construction)
# ---------------------------------------------------------------------------

def quantize_completed_kv_pages(key, value, key_center, value_center):
    """scripts/benchmark_page_gauge_overheads.py:23-83 (Triton bulk quantizer).

    Centered in float32 (not rounded to FP16), scale as the finalize, codes by
    sign-symmetric floor(q+0.5).  Inputs [pages,16,H,128] fp16, centers [H,128].
    Returns (key_codes, value_codes, key_scales, value_scales).
    """
    out = []
    for source, center in ((key, key_center), (value, value_center)):
        centered = f32(_as_f16(source).astype(np.float32) - _as_f16(center).astype(np.float32)[None, None])
        scale = page_scale(centered, axis=(1, 3))                     # [pages, H]
        quotient = f32(centered / scale.astype(np.float32)[:, None, :, None])
        out.append((sign_symmetric_round(quotient), scale))
    (key_codes, key_scales), (value_codes, value_scales) = out
    return key_codes, value_codes, key_scales, value_scales


def exact_center(values: np.ndarray) -> np.ndarray:
    """Per-(head,dim) mean over pages and tokens: fp16(fp32(exact_sum / n)).

    The reference takes ``values.float().mean(dim=(0,1)).half()``
    (scripts/benchmark_flashinfer_page_affine_int8.py:262); its float32
    reduction order is unspecified, so this build defines the mean from the
    exact sum (every fp16 value is an integer multiple of 2^-24, so the sum is
    exact in int64), divided in float64, rounded to float32, then to float16.
    """
    values = _as_f16(values)
    scaled = (values.astype(np.float64) * (2.0 ** 24)).astype(np.int64)
    total = scaled.sum(axis=(0, 1), dtype=np.int64)
    count = values.shape[0] * values.shape[1]
    mean = (total.astype(np.float64) * (2.0 ** -24)) / float(count)
    return mean.astype(np.float32).astype(np.float16)


def quantize_page_gauge(values: np.ndarray, center: Optional[np.ndarray] = None):
    """scripts/benchmark_flashinfer_page_affine_int8.py:256-278.

    Returns (codes, center, scale, reconstructed_centered, centered) exactly as
    the reference: codes use round-half-even of the float32 quotient.
    """
    values = _as_f16(values)
    if center is None:
        center = exact_center(values)
    centered32 = f32(values.astype(np.float32) - center.astype(np.float32)[None, None])
    scale = page_scale(centered32, axis=(1, 3))                          # [pages, H]
    quotient = f32(centered32 / scale.astype(np.float32)[:, None, :, None])
    codes = np.clip(np.rint(quotient), -127, 127).astype(np.int8)        # half-even
    reconstructed = f16(codes.astype(np.float32) * scale.astype(np.float32)[:, None, :, None])
    return codes, center, scale, reconstructed, centered32.astype(np.float16)


# ---------------------------------------------------------------------------
# A4/A5: decode attention and state merges
# ---------------------------------------------------------------------------

def _segment_tokens(pages_k, pages_v, scale_k, scale_v, indptr, indices, last_page_len,
                    request: int):
    """Gather one request's K/V tokens [T,Hkv,128] (float64) in logical order."""
    begin, end = int(indptr[request]), int(indptr[request + 1])
    if end <= begin:
        hkv = pages_k.shape[2]
        empty = np.zeros((0, hkv, DIM), dtype=np.float64)
        return empty, empty
    ids = np.asarray(indices[begin:end], dtype=np.int64)
    keys = pages_k[ids].astype(np.float64)             # [n,16,Hkv,128]
    vals = pages_v[ids].astype(np.float64)
    if scale_k is not None:
        keys = keys * scale_k[ids].astype(np.float64)[:, None, :, None]
        vals = vals * scale_v[ids].astype(np.float64)[:, None, :, None]
    last = int(last_page_len[request])
    n = ids.shape[0]
    keys = keys.reshape(n * PAGE, keys.shape[2], DIM)[: (n - 1) * PAGE + last]
    vals = vals.reshape(n * PAGE, vals.shape[2], DIM)[: (n - 1) * PAGE + last]
    return keys, vals


def attention_state(query, keys, values, sm_scale: float):
    """Unnormalised float64 state of one request: (o [Hq,128], lse [Hq]) base 2.

    Scores s = sm_scale * q.k in base 2 (FlashInfer convention: lse is
    log2-sum-exp2 of s*log2(e), tests/page_gauge_append_extension.cu:385-388).
    GQA: query head qh reads KV head qh // (Hq/Hkv).  Empty inputs give
    (o=0, lse=-inf).
    """
    hq = query.shape[0]
    hkv = keys.shape[1]
    group = hq // hkv
    q = query.astype(np.float64)
    out = np.zeros((hq, DIM), dtype=np.float64)
    lse = np.full((hq,), -np.inf, dtype=np.float64)
    if keys.shape[0] == 0:
        return out, lse
    for kv in range(hkv):
        qs = q[kv * group:(kv + 1) * group]                       # [g,128]
        scores = (qs @ keys[:, kv, :].T) * (sm_scale * LOG2E)      # [g,T]
        m = scores.max(axis=1, keepdims=True)
        w = np.exp2(scores - m)
        den = w.sum(axis=1, keepdims=True)
        out[kv * group:(kv + 1) * group] = (w @ values[:, kv, :]) / den
        lse[kv * group:(kv + 1) * group] = (np.log2(den) + m)[:, 0]
    return out, lse


def merge_state(o_a, lse_a, o_b, lse_b):
    """A5 base-2 state merge (tests/page_gauge_append_extension.cu:476-581)."""
    o_a = np.asarray(o_a, dtype=np.float64)
    o_b = np.asarray(o_b, dtype=np.float64)
    lse_a = np.asarray(lse_a, dtype=np.float64)
    lse_b = np.asarray(lse_b, dtype=np.float64)
    m = np.maximum(lse_a, lse_b)
    safe_m = np.where(np.isfinite(m), m, 0.0)
    w_a = np.exp2(lse_a - safe_m)
    w_b = np.exp2(lse_b - safe_m)
    den = w_a + w_b
    with np.errstate(invalid="ignore", divide="ignore"):
        o = (w_a[..., None] * o_a + w_b[..., None] * o_b) / den[..., None]
        lse = np.log2(den) + safe_m
    o = np.where(den[..., None] > 0, o, 0.0)
    lse = np.where(den > 0, lse, -np.inf)
    return o, lse


def decode(query, k_pages, v_pages, indptr, indices, last_page_len, sm_scale: float,
           k_scale=None, v_scale=None, tail_k=None, tail_v=None, tail_indptr=None,
           tail_indices=None, tail_last_page_len=None, value_center=None):
    """Dense float64 paged-decode reference (A4).

    ``k_pages``/``v_pages`` are INT8 codes when ``k_scale``/``v_scale`` are
    given (page-affine PageGauge pages: K = sK*Z) or FP16 pages otherwise.  The
    optional FP16 tail segment (centered ring pages) joins the same softmax;
    ``value_center`` ([B,Hkv,128] or [Hkv,128]) is added once after
    normalisation, repeated over the GQA group
    (scripts/benchmark_flashinfer_page_affine_int8.py:566-602,
    scripts/benchmark_page_gauge_transformer.py:345).  Returns
    (out float16 [B,Hq,128], lse float32 [B,Hq], out float64).
    """
    batch, hq, _ = query.shape
    hkv = k_pages.shape[2]
    group = hq // hkv
    outs = np.zeros((batch, hq, DIM), dtype=np.float64)
    lses = np.zeros((batch, hq), dtype=np.float64)
    for request in range(batch):
        keys, vals = _segment_tokens(k_pages, v_pages, k_scale, v_scale, indptr, indices,
                                     last_page_len, request)
        if tail_k is not None:
            tk, tv = _segment_tokens(tail_k, tail_v, None, None, tail_indptr, tail_indices,
                                     tail_last_page_len, request)
            keys = np.concatenate((keys, tk), axis=0)
            vals = np.concatenate((vals, tv), axis=0)
        o, lse = attention_state(query[request], keys, vals, sm_scale)
        if value_center is not None:
            center = _center_for(np.asarray(value_center), request).astype(np.float64)
            o = o + np.repeat(center, group, axis=0)
        outs[request] = o
        lses[request] = lse
    return outs.astype(np.float16), lses.astype(np.float32), outs


def decode_heterogeneous(query, k_codes, v_codes, k_scale, v_scale, exact_k, exact_v, indptr,
                         indices, last_page_len, old_kv_len, sm_scale: float, value_center=None):
    """One unified table per request (scripts/page_gauge_heterogeneous_fa2.py:336-381):
    entry j of request r indexes the INT8 code pool when j < old_kv_len[r]/16
    and the FP16 exact pages otherwise; the last entry holds last_page_len[r]
    tokens.  Restated as the segmented decode above (INT8 pages then the FP16
    pages of each request in one softmax)."""
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    batch = indptr.shape[0] - 1
    old_ptr, tail_ptr = [0], [0]
    old_idx, tail_idx, old_last, tail_last = [], [], [], []
    for r in range(batch):
        row = indices[indptr[r]:indptr[r + 1]]
        n_old = min(int(old_kv_len[r]) // PAGE, row.shape[0])
        old_idx.extend(row[:n_old])
        tail_idx.extend(row[n_old:])
        old_ptr.append(len(old_idx))
        tail_ptr.append(len(tail_idx))
        has_tail = row.shape[0] > n_old
        old_last.append(PAGE if has_tail else int(last_page_len[r]))
        tail_last.append(int(last_page_len[r]))
    return decode(query, k_codes, v_codes, np.array(old_ptr), np.array(old_idx, dtype=np.int64),
                  np.array(old_last), sm_scale, k_scale=k_scale, v_scale=v_scale, tail_k=exact_k,
                  tail_v=exact_v, tail_indptr=np.array(tail_ptr),
                  tail_indices=np.array(tail_idx, dtype=np.int64),
                  tail_last_page_len=np.array(tail_last), value_center=value_center)


def exact_tail_merge_center(query, exact_key_pages, exact_value_pages, exact_page_indices,
                            exact_last_page_len, old_output, old_lse, value_center,
                            sm_scale: float):
    """tests/page_gauge_append_extension.cu:389-583 in float64.

    Tail of ``(n-1)*16 + last_len[r]`` tokens read through
    ``exact_page_indices[r*n:(r+1)*n]``; merged with the old normalised state
    ``(old_output, old_lse)`` and ``value_center`` added.  Returns the new
    (output float16, lse float32).
    """
    batch, hq, _ = query.shape
    n = exact_page_indices.shape[0] // batch
    indptr = np.arange(batch + 1) * n
    out = np.zeros_like(old_output, dtype=np.float16)
    lse_out = np.zeros((batch, hq), dtype=np.float32)
    hkv = exact_key_pages.shape[2]
    group = hq // hkv
    for request in range(batch):
        keys, vals = _segment_tokens(exact_key_pages, exact_value_pages, None, None, indptr,
                                     exact_page_indices, exact_last_page_len, request)
        o_t, lse_t = attention_state(query[request], keys, vals, sm_scale)
        o, lse = merge_state(old_output[request].astype(np.float64),
                             old_lse[request].astype(np.float64), o_t, lse_t)
        center = _center_for(np.asarray(value_center), request).astype(np.float64)
        out[request] = (o + np.repeat(center, group, axis=0)).astype(np.float16)
        lse_out[request] = lse.astype(np.float32)
    return out, lse_out


def merge_state_in_place(v, s, v_other, s_other, mask=None):
    """flashinfer.merge_state_in_place restated: returns new (v fp16, s fp32)."""
    o, lse = merge_state(v.astype(np.float64), s.astype(np.float64),
                         v_other.astype(np.float64), s_other.astype(np.float64))
    o = o.astype(np.float16)
    lse = lse.astype(np.float32)
    if mask is not None:
        keep = ~np.asarray(mask, dtype=bool)
        o[keep] = v[keep]
        lse[keep] = s[keep]
    return o, lse


# ---------------------------------------------------------------------------
# RoPE tables (scripts/benchmark_page_gauge_transformer.py:3629-3636)
# ---------------------------------------------------------------------------

def rope_tables(positions: int, theta: float = 1.0e6, dim: int = DIM):
    """HF Mistral rotary tables: float32 angles -> cos/sin -> fp16 [positions,128]."""
    inv_freq = (1.0 / (np.float32(theta) ** (np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim)))).astype(np.float32)
    t = np.arange(positions, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    emb = np.concatenate((freqs, freqs), axis=-1)
    return np.cos(emb).astype(np.float32).astype(np.float16), np.sin(emb).astype(np.float32).astype(np.float16)


__all__ = [name for name in dir() if not name.startswith("_")]
