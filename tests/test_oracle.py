"""Pins of the CPU oracle (``oracle/pg_oracle.py`` and ``oracle/pg_oracle.c``).

Each oracle function is checked against something it is not a retyping of:
the reference tests' own torch formulas evaluated by torch on the CPU, exact
rational arithmetic (``fractions``), closed-form special cases, algebraic
invariants of attention, and the independent C restatement.  Every check is
chosen so that a plausible mistake (a dropped term, a sign, a half-even
instead of half-away rounding, a transposed operand) fails it.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import pg_oracle as oracle

RNG = np.random.default_rng(20260840)


def _f16(shape, scale=1.0, rng=RNG):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a.view(np.uint8),
                                                                        b.view(np.uint8))


# ---------------------------------------------------------------------------
# A1 RoPE
# ---------------------------------------------------------------------------

def test_rope_matches_reference_torch_fp16_formula():
    """tests/test_page_gauge_append_extension.py:77-84, evaluated by torch on the CPU.

    torch rounds each fp16 op once through float32; float32 has 24 >= 2*11+2
    bits, so that double rounding equals one correct fp16 rounding, exactly
    what the kernel's mul.rn.f16/add.rn.f16 sequence produces.
    """
    cos_t, sin_t = oracle.rope_tables(5000)
    x = _f16((6, 32, 128), 3.0)
    for position in (0, 1, 17, 4095, 4999):
        c, s = cos_t[position], sin_t[position]
        got = oracle.rope_rotate(x, c, s)
        tx, tc, ts = torch.from_numpy(x), torch.from_numpy(c), torch.from_numpy(s)
        want = tx * tc + torch.cat((-tx[..., 64:], tx[..., :64]), dim=-1) * ts
        assert _bits_equal(got, want.numpy()), position


def test_rope_identity_and_quarter_turn():
    """cos=1, sin=0 is the identity; cos=0, sin=1 is the pure rotate-half."""
    x = _f16((4, 8, 128), 2.0)
    one, zero = np.ones(128, np.float16), np.zeros(128, np.float16)
    assert _bits_equal(oracle.rope_rotate(x, one, zero), x + np.float16(0))
    turned = oracle.rope_rotate(x, zero, one)
    assert _bits_equal(turned[..., :64], (-x[..., 64:]) + np.float16(0))
    assert _bits_equal(turned[..., 64:], x[..., :64] + np.float16(0))


def test_rope_tables_match_transformers_rotary_embedding():
    """Tables follow HF Mistral rotary_emb (scripts/benchmark_page_gauge_transformer.py:3629-3636)."""
    transformers = pytest.importorskip("transformers")
    config = transformers.MistralConfig(hidden_size=4096, num_attention_heads=32,
                                        num_key_value_heads=8, head_dim=128, rope_theta=1.0e6,
                                        max_position_embeddings=32768)
    rotary = transformers.models.mistral.modeling_mistral.MistralRotaryEmbedding(config=config)
    positions = torch.arange(4096)[None]
    probe = torch.empty(1, 1, 4096, dtype=torch.float16)
    cos, sin = rotary(probe, positions)
    cos, sin = cos[0].to(torch.float16).numpy(), sin[0].to(torch.float16).numpy()
    ours_cos, ours_sin = oracle.rope_tables(4096)
    for ours, theirs in ((ours_cos, cos), (ours_sin, sin)):
        diff = np.abs(ours.astype(np.float64) - theirs.astype(np.float64))
        # float32 pow/cos implementations may differ by an ulp before the fp16 rounding
        assert diff.max() <= 2.0 ** -10
        assert (diff == 0).mean() > 0.99


def test_c_rope_equals_numpy_rope():
    cos_t, sin_t = oracle.rope_tables(64)
    x = _f16((3, 40, 128), 4.0)
    for position in (0, 31, 63):
        got = c_oracle.rope_rotate(x, cos_t[position], sin_t[position])
        assert _bits_equal(got, oracle.rope_rotate(x, cos_t[position], sin_t[position]))


# ---------------------------------------------------------------------------
# A3 scale and sign-symmetric rounding
# ---------------------------------------------------------------------------

def _rn32_exact(value: Fraction) -> np.float32:
    # float(Fraction) is correctly rounded to binary64; 53 >= 2*24+2 makes the
    # second rounding to binary32 innocuous.
    return np.float32(float(value))


def _sign_symmetric_exact(q: np.float32) -> int:
    fq = Fraction(float(q))
    if q >= 0:
        r = math.floor(Fraction(float(_rn32_exact(fq + Fraction(1, 2)))))
    else:
        r = -math.floor(Fraction(float(_rn32_exact(-fq + Fraction(1, 2)))))
    return max(-127, min(127, r))


def test_sign_symmetric_round_brute_force():
    specials = [0.0, -0.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 127.49, 127.5, 200.0,
                -300.0, 0.49999997, -0.49999997, np.nextafter(np.float32(0.5), np.float32(0)),
                np.nextafter(np.float32(2.5), np.float32(0)), 1e-30, -1e-30, 8388607.5]
    q = np.concatenate([np.array(specials, dtype=np.float32),
                        (RNG.standard_normal(4000) * 60).astype(np.float32),
                        (RNG.integers(-300, 300, 2000) + 0.5).astype(np.float32)])
    got = oracle.sign_symmetric_round(q)
    want = np.array([_sign_symmetric_exact(v) for v in q], dtype=np.int8)
    assert np.array_equal(got, want)
    # the reference's quirk: rn32(q + 0.5) rounds 0.5 - 2^-25 up to 1.0
    assert oracle.sign_symmetric_round(np.array([0.5 - 2.0 ** -25], np.float32))[0] == 1
    # half-away, not half-even
    assert list(oracle.sign_symmetric_round(np.array([2.5, -2.5, 0.5], np.float32))) == [3, -3, 1]


def test_float32_division_is_correctly_rounded():
    num = (RNG.standard_normal(3000) * 10).astype(np.float16).astype(np.float32)
    den = np.abs(RNG.standard_normal(3000)).astype(np.float16).astype(np.float32) + np.float32(1e-3)
    got = (num / den).astype(np.float32)
    want = np.array([_rn32_exact(Fraction(float(a)) / Fraction(float(b)))
                     for a, b in zip(num, den)], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_page_scale_matches_reference_torch_formula():
    """tests/test_page_gauge_overheads.py:54-63: (amax/127).clamp_min(2^-20).half()."""
    values = (RNG.standard_normal((5, 16, 8, 128)) * np.array([1e-7, 1e-3, 1, 30, 1e4])
              [:, None, None, None]).astype(np.float32)
    values[2, :, 3] = 0.0                                  # an all-zero (page, head) block
    got = oracle.page_scale(values, axis=(1, 3))
    want = (torch.from_numpy(values).permute(0, 2, 1, 3).abs().amax(dim=(2, 3)).div(127.0)
            .clamp_min(2.0 ** -20).half().numpy())
    assert _bits_equal(got, want)
    assert got[2, 3] == np.float16(2.0 ** -20)


# ---------------------------------------------------------------------------
# Bulk quantizers
# ---------------------------------------------------------------------------

def _torch_quantize_completed(values: np.ndarray, center: np.ndarray):
    """Torch transcription of scripts/benchmark_page_gauge_overheads.py:23-83."""
    centered = torch.from_numpy(values).float() - torch.from_numpy(center).float()[None, None]
    scale = (centered.abs().amax(dim=(1, 3)) / 127.0).clamp_min(2.0 ** -20).half()
    quotient = centered / scale.float()[:, None, :, None]
    rounded = torch.where(quotient >= 0, torch.floor(quotient + 0.5), -torch.floor(-quotient + 0.5))
    return rounded.clamp(-127, 127).to(torch.int8).numpy(), scale.numpy()


def test_quantize_completed_kv_pages_matches_torch_transcription():
    key = _f16((6, 16, 4, 128), 1.5)
    value = _f16((6, 16, 4, 128), 0.7)
    kc, vc = _f16((4, 128), 0.2), _f16((4, 128), 0.2)
    key_codes, value_codes, key_scales, value_scales = oracle.quantize_completed_kv_pages(
        key, value, kc, vc)
    for codes, scales, src, center in ((key_codes, key_scales, key, kc),
                                       (value_codes, value_scales, value, vc)):
        want_codes, want_scales = _torch_quantize_completed(src, center)
        assert _bits_equal(scales, want_scales)
        assert np.array_equal(codes, want_codes)
        recon = codes.astype(np.float32) * scales.astype(np.float32)[:, None, :, None] + \
            center.astype(np.float32)[None, None]
        rel = np.linalg.norm(recon - src.astype(np.float32)) / np.linalg.norm(src.astype(np.float32))
        assert rel < 0.02
        c_codes, c_scales = c_oracle.quantize_completed(src, center)
        assert np.array_equal(c_codes, codes) and _bits_equal(c_scales, scales)


def _torch_quantize_page_gauge(values: np.ndarray):
    """Torch transcription of scripts/benchmark_flashinfer_page_affine_int8.py:256-278."""
    v = torch.from_numpy(values)
    center = v.float().mean(dim=(0, 1)).half()
    centered = v.float() - center.float()[None, None]
    page_head = centered.permute(0, 2, 1, 3)
    scale = (page_head.abs().amax(dim=(2, 3)) / 127.0).clamp_min(2.0 ** -20).half()
    codes = ((page_head / scale.float()[:, :, None, None]).round().clamp(-127, 127)
             .to(torch.int8).permute(0, 2, 1, 3).contiguous())
    return codes.numpy(), center.numpy(), scale.numpy()


def test_quantize_page_gauge_matches_torch_transcription():
    values = _f16((7, 16, 8, 128), 1.0)
    codes, center, scale, recon, centered = oracle.quantize_page_gauge(values)
    want_codes, want_center, want_scale = _torch_quantize_page_gauge(values)
    # the center is defined from the exact sum; torch's float32 reduction may
    # land one fp16 ulp away in rare ties
    diff = np.abs(center.astype(np.float64) - want_center.astype(np.float64))
    assert (diff == 0).mean() > 0.99
    assert diff.max() <= np.abs(np.spacing(want_center.astype(np.float16))).max()
    # with the same center, scales and codes are bit-exact
    codes2, _, scale2, _, _ = oracle.quantize_page_gauge(values, center=want_center)
    assert _bits_equal(scale2, want_scale)
    assert np.array_equal(codes2, want_codes)
    rel = np.linalg.norm(recon.astype(np.float64) - centered.astype(np.float64)) / \
        np.linalg.norm(centered.astype(np.float64))
    assert rel < 0.02                             # tests/test_flashinfer_page_affine_int8.py:46


def test_quantize_page_gauge_rounds_half_even():
    """The torch quantizer uses round-half-even, unlike the kernels' half-away rule."""
    values = np.zeros((1, 16, 8, 128), np.float16)
    values[0, 0, 0, 0] = 127.0     # amax 127 -> scale 1
    values[0, 1, 0, 0] = 2.5
    values[0, 2, 0, 0] = -2.5
    values[0, 3, 0, 0] = 3.5
    codes, *_ = oracle.quantize_page_gauge(values, center=np.zeros((8, 128), np.float16))
    assert list(codes[0, :4, 0, 0]) == [127, 2, -2, 4]
    completed, *_ = oracle.quantize_completed_kv_pages(values, values, np.zeros((8, 128), np.float16),
                                                       np.zeros((8, 128), np.float16))
    assert list(completed[0, :4, 0, 0]) == [127, 3, -3, 4]


def test_exact_center_is_the_exact_mean():
    values = _f16((9, 16, 2, 128), 2.0)
    got = oracle.exact_center(values)
    exact = [[float(sum(Fraction(float(v)) for v in values[:, :, h, d].ravel()) / (9 * 16))
              for d in range(0, 128, 17)] for h in range(2)]
    want = np.array(exact, dtype=np.float64).astype(np.float32).astype(np.float16)
    assert _bits_equal(got[:, ::17], want)


# ---------------------------------------------------------------------------
# K2 append / finalize placement and equivalences
# ---------------------------------------------------------------------------

def test_finalize_codes_c_and_numpy_agree_and_reconstruct():
    page = _f16((16, 8, 128), 0.8)
    page[:, 2] = 0                                    # zero head: scale 2^-20, codes 0
    codes, scales = oracle.finalize_codes(page, axis=(0, 2))
    c_codes, c_scales = c_oracle.finalize_page(page)
    assert np.array_equal(codes, c_codes) and _bits_equal(scales, c_scales)
    assert scales[2] == np.float16(2.0 ** -20) and not codes[:, 2].any()
    assert np.abs(codes).max() == 127
    recon = codes.astype(np.float32) * scales.astype(np.float32)[None, :, None]
    assert np.abs(recon - page.astype(np.float32)).max() <= scales.astype(np.float32).max() * 0.5001


def _fresh_page_gauge_buffers(batch, ring_per_request, code_pages_per_request):
    return dict(
        rotated_query=np.zeros((batch, 32, 128), np.float16),
        exact_key_pages=np.zeros((batch * ring_per_request, 16, 8, 128), np.float16),
        exact_value_pages=np.zeros((batch * ring_per_request, 16, 8, 128), np.float16),
        key_codes=np.zeros((batch * code_pages_per_request, 16, 8, 128), np.int8),
        value_codes=np.zeros((batch * code_pages_per_request, 16, 8, 128), np.int8),
        key_scales=np.zeros((batch * code_pages_per_request, 8), np.float16),
        value_scales=np.zeros((batch * code_pages_per_request, 8), np.float16),
    )


@pytest.mark.parametrize("sink", [0, 1, 3])
def test_ring_slot_placement_matches_host_exact_page_table(sink):
    """Kernel ring slot req*E + (page<S ? page : S + page%(E-S))
    (tests/page_gauge_append_extension.cu:288-293) equals the decoder's
    request_major_exact_page_table (scripts/benchmark_page_gauge_transformer.py:492-524)."""
    from pagegauge_amd.page_table import request_major_exact_page_table

    batch, tail, code_pages = 2, 4, 12
    ring = sink + tail
    table = request_major_exact_page_table(batch, code_pages, tail, sink, device="cpu").numpy()
    cos, sin = np.ones(128, np.float16), np.zeros(128, np.float16)
    centers = np.zeros((batch, 8, 128), np.float16)
    for position in range(0, code_pages * 16, 16):
        buf = _fresh_page_gauge_buffers(batch, ring, code_pages)
        key = np.ones((batch, 8, 128), np.float16)
        oracle.rope_append_page_gauge(np.zeros((batch, 32, 128), np.float16), key, key, cos, sin,
                                      centers, centers, exact_sink_pages=sink, position=position,
                                      **buf)
        written = sorted(set(np.flatnonzero(buf["exact_key_pages"].reshape(batch * ring, -1).any(1))))
        page = position // 16
        assert written == [int(table[r, page]) for r in range(batch)]


def test_page_gauge_append_closes_page_into_codes():
    """Sixteen appends fill one ring page; the last one writes codes/scales of
    code page req*Pc + page (:327-382) equal to finalize_codes of the ring page."""
    batch, ring, code_pages = 2, 3, 4
    cos_t, sin_t = oracle.rope_tables(64)
    kc, vc = _f16((batch, 8, 128), 0.1), _f16((batch, 8, 128), 0.1)
    buf = _fresh_page_gauge_buffers(batch, ring, code_pages)
    keys, values = _f16((64, batch, 8, 128)), _f16((64, batch, 8, 128))
    query = _f16((batch, 32, 128))
    for position in range(16, 32):
        oracle.rope_append_page_gauge(query, keys[position], values[position], cos_t[position],
                                      sin_t[position], kc, vc, exact_sink_pages=1,
                                      position=position, **buf)
        if position < 31:
            assert not buf["key_codes"].any()
    for r in range(batch):
        slot = r * ring + 1 + 1 % (ring - 1)
        rotated = oracle.rope_rotate(keys[16:32, r], cos_t[16:32, None, :], sin_t[16:32, None, :])
        centered = oracle.f16(rotated.astype(np.float32) - kc[r].astype(np.float32))
        assert _bits_equal(buf["exact_key_pages"][slot], centered)
        codes, scales = oracle.finalize_codes(centered, axis=(0, 2))
        assert np.array_equal(buf["key_codes"][r * code_pages + 1], codes)
        assert _bits_equal(buf["key_scales"][r * code_pages + 1], scales)
        # tests/test_page_gauge_append_extension.py reconstruction bound
        recon = codes.astype(np.float32) * scales.astype(np.float32)[None, :, None]
        rel = np.linalg.norm(recon - centered.astype(np.float32)) / np.linalg.norm(centered.astype(np.float32))
        assert rel < 0.02
    assert _bits_equal(buf["rotated_query"], oracle.rope_rotate(query, cos_t[31], sin_t[31]))


def test_append_finalize_equals_page_gauge_append_at_identity_rope():
    batch, pages = 2, 2
    kc, vc = _f16((8, 128), 0.1), _f16((8, 128), 0.1)
    keys, values = _f16((32, batch, 8, 128)), _f16((32, batch, 8, 128))
    cos, sin = np.ones(128, np.float16), np.zeros(128, np.float16)
    a = _fresh_page_gauge_buffers(batch, pages, pages)
    b = _fresh_page_gauge_buffers(batch, pages, pages)
    for position in range(32):
        oracle.rope_append_page_gauge(np.zeros((batch, 32, 128), np.float16), keys[position],
                                      values[position], cos, sin, np.stack([kc] * batch),
                                      np.stack([vc] * batch), exact_sink_pages=0,
                                      position=position, **a)
        page, token = divmod(position, 16)
        ids = np.array([r * pages + page for r in range(batch)], np.int32)
        oracle.append_finalize_page_gauge(keys[position], values[position], kc, vc,
                                          b["exact_key_pages"], b["exact_value_pages"],
                                          b["key_codes"], b["value_codes"], b["key_scales"],
                                          b["value_scales"], ids, np.full(batch, token, np.int32))
    for name in ("exact_key_pages", "exact_value_pages", "key_codes", "value_codes", "key_scales",
                 "value_scales"):
        assert _bits_equal(a[name], b[name]), name


def test_positions_variant_equals_scalar_kernel_row_by_row():
    batch, ring, code_pages = 3, 2, 3
    cos_t, sin_t = oracle.rope_tables(48)
    kc, vc = _f16((batch, 8, 128), 0.1), _f16((batch, 8, 128), 0.1)
    positions = np.array([15, 20, 47], np.int32)
    query, key, value = _f16((batch, 32, 128)), _f16((batch, 8, 128)), _f16((batch, 8, 128))
    a = _fresh_page_gauge_buffers(batch, ring, code_pages)
    oracle.rope_append_page_gauge_positions(query, key, value, cos_t, sin_t, positions, kc, vc,
                                            exact_sink_pages=0, **a)
    for r in range(batch):
        b = _fresh_page_gauge_buffers(batch, ring, code_pages)
        oracle.rope_append_page_gauge(query, key, value, cos_t[positions[r]], sin_t[positions[r]],
                                      kc, vc, exact_sink_pages=0, position=int(positions[r]), **b)
        assert _bits_equal(a["rotated_query"][r], b["rotated_query"][r])
        for name in ("exact_key_pages", "key_codes", "key_scales"):
            rows = slice(r * b[name].shape[0] // batch, (r + 1) * b[name].shape[0] // batch)
            assert _bits_equal(a[name][rows], b[name][rows]), name


def test_slots_variant_equals_positions_variant_on_request_major_ids():
    """rope_append_page_gauge_slots with the request-major ids that the
    positions variant derives (exact page r*E + ring slot of the position's
    page, code page r*P + page) writes exactly what the positions variant
    writes, over 40 steps with ring wraps and finalizes; a row whose id is
    negative or outside the pool is skipped."""
    batch, ring, code_pages, sink = 3, 3, 6, 1
    cos_t, sin_t = oracle.rope_tables(code_pages * 16)
    kc, vc = _f16((batch, 8, 128), 0.1), _f16((batch, 8, 128), 0.1)
    a = _fresh_page_gauge_buffers(batch, ring, code_pages)
    b = _fresh_page_gauge_buffers(batch, ring, code_pages)
    start = np.array([0, 7, 30], np.int32)
    for step in range(40):
        query, key, value = _f16((batch, 32, 128)), _f16((batch, 8, 128)), _f16((batch, 8, 128))
        pos = start + step
        pages = pos // 16
        local = np.where(pages < sink, pages, sink + pages % (ring - sink))
        exact_ids = np.arange(batch) * ring + local
        code_ids = np.arange(batch) * code_pages + pages
        oracle.rope_append_page_gauge_positions(query, key, value, cos_t, sin_t, pos, kc, vc,
                                                exact_sink_pages=sink, **a)
        oracle.rope_append_page_gauge_slots(query, key, value, cos_t, sin_t, pos, exact_ids,
                                            code_ids, kc, vc, **b)
    for name in a:
        assert _bits_equal(a[name], b[name]), name
    assert np.abs(a["key_scales"]).max() > 0
    before = {k: v.copy() for k, v in b.items()}
    oracle.rope_append_page_gauge_slots(query, key, value, cos_t, sin_t, pos,
                                        np.array([-1, batch * ring, 0]), np.array([0, 0, -1]),
                                        kc, vc, **b)
    for name in b:
        if name != "rotated_query":
            assert _bits_equal(b[name], before[name]), name


def test_append_kv_against_the_fused_append_relation():
    """The reference's own cross-check of its two appends
    (scripts/benchmark_page_gauge_overheads.py:556-609): after one 16-step
    cycle at offsets 0..15, the fused append's exact pages plus the center
    equal the plain append's pages within 2e-3 (one FP16 rounding of the
    centered value), and its codes reconstruct them with relative L2 < 0.03.
    The plain append is also the FP16 append at identity RoPE placed at
    (page_ids, offsets)."""
    batch, heads = 3, 2
    page_ids = np.array([4, 0, 2], np.int32)
    kc, vc = _f16((heads, 128), 0.1), _f16((heads, 128), 0.1)
    plain = [np.zeros((6, 16, heads, 128), np.float16) for _ in range(2)]
    fused = [np.zeros((6, 16, heads, 128), np.float16) for _ in range(2)]
    fused += [np.zeros((6, 16, heads, 128), np.int8) for _ in range(2)]
    fused += [np.zeros((6, heads), np.float16) for _ in range(2)]
    keys = [_f16((batch, heads, 128)) for _ in range(16)]
    values = [_f16((batch, heads, 128)) for _ in range(16)]
    for t in range(16):
        offsets = np.full(batch, t, np.int32)
        oracle.append_kv(keys[t], values[t], *plain, page_ids, offsets)
        oracle.append_finalize_page_gauge(keys[t], values[t], kc, vc, *fused, page_ids, offsets)
    for r, page in enumerate(page_ids):
        for t in range(16):
            assert _bits_equal(plain[0][page, t], keys[t][r])
            assert _bits_equal(plain[1][page, t], values[t][r])
    exact = fused[0][page_ids].astype(np.float32) + kc.astype(np.float32)
    assert np.abs(exact - plain[0][page_ids].astype(np.float32)).max() <= 2e-3
    recon = (fused[2][page_ids].astype(np.float32) * fused[4][page_ids].astype(np.float32)[:, None, :, None]
             + kc.astype(np.float32))
    base = plain[0][page_ids].astype(np.float32)
    assert np.linalg.norm(recon - base) / np.linalg.norm(base) < 0.03
    untouched = [p for p in range(6) if p not in page_ids]
    assert not plain[0][untouched].any()


@pytest.mark.parametrize("seed", range(6))
def test_decode_fuzzed_page_tables(seed):
    """Random ragged tables over one shared, shuffled pool (empty requests,
    single pages, partial last pages, shared physical pages): the oracle's
    paged decode equals the dense softmax over the tokens gathered page by
    page in table order, and is invariant to renumbering the pool."""
    rng = np.random.default_rng(1000 + seed)
    batch = int(rng.integers(1, 5))
    pool = int(rng.integers(2, 12))
    k, v, ks, vs = _random_paged(pool, seed)
    counts = rng.integers(0, 5, batch)
    indptr = np.concatenate(([0], np.cumsum(counts))).astype(np.int32)
    indices = rng.integers(0, pool, int(indptr[-1])).astype(np.int32)   # pages may repeat
    last = rng.integers(1, 17, batch).astype(np.int32)
    q = _f16((batch, 32, 128), 0.4)
    out, lse, out64 = oracle.decode(q, k, v, indptr, indices, last, 128 ** -0.5, k_scale=ks,
                                    v_scale=vs)
    for r in range(batch):
        ids = indices[indptr[r]:indptr[r + 1]]
        if ids.size == 0:
            assert np.isneginf(lse[r]).all() and not out64[r].any()
            continue
        keys = (k[ids].astype(np.float64) * ks[ids].astype(np.float64)[:, None, :, None])
        vals = (v[ids].astype(np.float64) * vs[ids].astype(np.float64)[:, None, :, None])
        n = (ids.size - 1) * 16 + int(last[r])
        keys = keys.reshape(-1, 8, 128)[:n]
        vals = vals.reshape(-1, 8, 128)[:n]
        for h in range(32):
            s = keys[:, h // 4] @ q[r, h].astype(np.float64) * 128 ** -0.5
            p = np.exp(s - s.max())
            assert np.allclose(out64[r, h], p @ vals[:, h // 4] / p.sum(), atol=1e-9)
            assert abs(lse[r, h] - (np.log(p.sum()) + s.max()) / np.log(2)) < 1e-4
    perm = rng.permutation(pool)
    inverse = np.argsort(perm)
    out2, _, _ = oracle.decode(q, k[perm], v[perm], indptr, inverse[indices].astype(np.int32), last,
                               128 ** -0.5, k_scale=ks[perm], v_scale=vs[perm])
    assert _bits_equal(out, out2)


def test_rope_append_fp16_request_major_placement():
    """Identity RoPE + page request*P + position//16 (tests/test_page_gauge_append_extension.py:766-786)."""
    batch, pages = 3, 3
    kp = np.zeros((batch * pages, 16, 8, 128), np.float16)
    vp = np.zeros_like(kp)
    rq = np.zeros((batch, 32, 128), np.float16)
    key, value = _f16((batch, 8, 128)), _f16((batch, 8, 128))
    query = _f16((batch, 32, 128))
    oracle.rope_append_fp16(query, key, value, np.ones(128, np.float16), np.zeros(128, np.float16),
                            rq, kp, vp, position=37)
    for r in range(batch):
        assert _bits_equal(kp[r * pages + 2, 5], key[r] + np.float16(0))
        assert _bits_equal(vp[r * pages + 2, 5], value[r])
    assert np.count_nonzero(kp.reshape(batch * pages * 16, -1).any(1)) == batch
    # out-of-range position: a silent no-op (tests/page_gauge_append_extension.cu:203-207)
    before = kp.copy()
    oracle.rope_append_fp16(query, key, value, np.ones(128, np.float16), np.zeros(128, np.float16),
                            rq, kp, vp, position=pages * 16)
    assert _bits_equal(kp, before)


# ---------------------------------------------------------------------------
# A4/A5 decode, merge, tail
# ---------------------------------------------------------------------------

def _random_paged(pages, seed):
    rng = np.random.default_rng(seed)
    k_codes = rng.integers(-127, 128, (pages, 16, 8, 128)).astype(np.int8)
    v_codes = rng.integers(-127, 128, (pages, 16, 8, 128)).astype(np.int8)
    k_scale = (rng.random((pages, 8)) * 0.02 + 1e-3).astype(np.float16)
    v_scale = (rng.random((pages, 8)) * 0.02 + 1e-3).astype(np.float16)
    return k_codes, v_codes, k_scale, v_scale


def test_decode_matches_torch_float64_softmax():
    """Dense reference of diagnostics/benchmark_heterogeneous_fa2_correctness.py:291-299 in float64."""
    k_codes, v_codes, k_scale, v_scale = _random_paged(20, 1)
    perm = np.random.default_rng(2).permutation(20).astype(np.int32)
    indptr = np.array([0, 7, 7, 20], np.int32)                    # one empty request
    last = np.array([5, 16, 16], np.int32)
    q = _f16((3, 32, 128))
    sm_scale = 1.0 / math.sqrt(128)
    out, lse, out64 = oracle.decode(q, k_codes, v_codes, indptr, perm, last, sm_scale,
                                    k_scale=k_scale, v_scale=v_scale)
    for r in (0, 2):
        ids = perm[indptr[r]:indptr[r + 1]]
        k = torch.from_numpy(k_codes[ids]).double() * torch.from_numpy(k_scale[ids]).double()[:, None, :, None]
        v = torch.from_numpy(v_codes[ids]).double() * torch.from_numpy(v_scale[ids]).double()[:, None, :, None]
        tokens = (len(ids) - 1) * 16 + int(last[r])
        k = k.reshape(-1, 8, 128)[:tokens].repeat_interleave(4, dim=1)
        v = v.reshape(-1, 8, 128)[:tokens].repeat_interleave(4, dim=1)
        score = torch.einsum("hd,thd->ht", torch.from_numpy(q[r]).double(), k) * sm_scale
        want = torch.einsum("ht,thd->hd", torch.softmax(score, dim=-1), v)
        np.testing.assert_allclose(out64[r], want.numpy(), rtol=0, atol=1e-12)
        want_lse = torch.logsumexp(score, dim=-1) / math.log(2.0)
        np.testing.assert_allclose(lse[r], want_lse.numpy(), rtol=1e-6, atol=1e-6)
    assert not out64[1].any() and np.all(np.isneginf(lse[1]))


def test_decode_merge_associativity_and_value_center():
    """decode(A u B) = merge(decode(A), decode(B)); the value center adds once."""
    k_codes, v_codes, k_scale, v_scale = _random_paged(12, 3)
    q = _f16((1, 32, 128))
    s = 1.0 / math.sqrt(128)
    idx = np.arange(12, dtype=np.int32)
    full = oracle.decode(q, k_codes, v_codes, np.array([0, 12], np.int32), idx,
                         np.array([16], np.int32), s, k_scale=k_scale, v_scale=v_scale)
    a = oracle.decode(q, k_codes, v_codes, np.array([0, 5], np.int32), idx,
                      np.array([16], np.int32), s, k_scale=k_scale, v_scale=v_scale)
    b = oracle.decode(q, k_codes, v_codes, np.array([0, 7], np.int32), idx[5:],
                      np.array([16], np.int32), s, k_scale=k_scale, v_scale=v_scale)
    o, lse = oracle.merge_state(a[2], a[1].astype(np.float64), b[2], b[1].astype(np.float64))
    np.testing.assert_allclose(o, full[2], atol=1e-6)
    np.testing.assert_allclose(lse, full[1], atol=1e-5)
    center = _f16((1, 8, 128), 0.3)
    with_c = oracle.decode(q, k_codes, v_codes, np.array([0, 12], np.int32), idx,
                           np.array([16], np.int32), s, k_scale=k_scale, v_scale=v_scale,
                           value_center=center)
    np.testing.assert_allclose((with_c[2] - full[2])[0], np.repeat(center[0].astype(np.float64), 4, 0),
                               atol=1e-12)


def test_decode_key_center_is_a_softmax_gauge():
    """tests/test_gauge_int8_model.py:20-27: shifting every key by one vector
    leaves the softmax unchanged (FP16 pages path)."""
    keys = _f16((64, 8, 128), 0.5).astype(np.float64)
    vals = _f16((64, 8, 128), 0.5).astype(np.float64)
    shift = _f16((8, 128), 0.5).astype(np.float64)
    q = _f16((32, 128))
    a = oracle.attention_state(q, keys, vals, 0.088)
    b = oracle.attention_state(q, keys + shift, vals, 0.088)
    np.testing.assert_allclose(a[0], b[0], atol=1e-12)
    # the lse moves by exactly q.shift * sm_scale * log2(e) per query head
    moved = (q.astype(np.float64) @ np.repeat(shift, 4, 0).T).diagonal() * 0.088 * oracle.LOG2E
    np.testing.assert_allclose(b[1] - a[1], moved, atol=1e-9)


def test_merge_state_closed_forms():
    o = np.random.default_rng(5).standard_normal((2, 4, 128))
    lse = np.array([[1.0, 2.0, -np.inf, 3.0], [0.5, 0.5, 7.0, -np.inf]])
    finite = np.isfinite(lse)
    o2, lse2 = oracle.merge_state(o, lse, o, lse)
    np.testing.assert_allclose(o2[finite], o[finite], atol=1e-12)   # a state merged with itself
    np.testing.assert_allclose(lse2[finite], lse[finite] + 1.0)
    assert not o2[~finite].any() and np.all(np.isneginf(lse2[~finite]))  # two empty states
    empty = np.full((2, 4), -np.inf)
    o3, lse3 = oracle.merge_state(o, lse, np.zeros_like(o), empty)
    np.testing.assert_allclose(o3[finite], o[finite], atol=1e-12)
    assert np.array_equal(np.isneginf(lse3), ~finite)


def test_merge_state_in_place_mask():
    v = _f16((3, 4, 128))
    s = np.zeros((3, 4), np.float32)
    v2 = _f16((3, 4, 128))
    s2 = np.full((3, 4), 50.0, np.float32)
    mask = np.array([1, 0, 1], bool)
    o, lse = oracle.merge_state_in_place(v, s, v2, s2, mask)
    assert _bits_equal(o[1], v[1]) and _bits_equal(lse[1], s[1])
    np.testing.assert_allclose(o[0].astype(np.float64), v2[0].astype(np.float64), atol=1e-3)


def _reference_tail_oracle(query, exact_key, exact_value, indices, tail_tokens, old_output,
                           old_lse, value_center, sm_scale):
    """torch transcription of tests/test_page_gauge_append_extension.py:628-657 (CPU float32)."""
    hq, hkv = query.shape[0], exact_key.shape[2]
    log2_e = 1.4426950408889634
    q = torch.from_numpy(query).float()
    k = torch.from_numpy(exact_key)[torch.from_numpy(indices).long()].reshape(-1, hkv, 128)[:tail_tokens].float()
    v = torch.from_numpy(exact_value)[torch.from_numpy(indices).long()].reshape(-1, hkv, 128)[:tail_tokens].float()
    kv_for_query = torch.arange(hq) // (hq // hkv)
    scores = torch.einsum("qd,qtd->qt", q, k[:, kv_for_query].permute(1, 0, 2)) * (sm_scale * log2_e)
    old_lse_t = torch.from_numpy(old_lse).float()
    merged_max = torch.maximum(old_lse_t, scores.amax(dim=1))
    old_weight = torch.exp2(old_lse_t - merged_max)
    tail_weight = torch.exp2(scores - merged_max[:, None])
    den = old_weight + tail_weight.sum(dim=1)
    ref = (old_weight[:, None] * torch.from_numpy(old_output).float()
           + torch.einsum("qt,qtd->qd", tail_weight, v[:, kv_for_query].permute(1, 0, 2))) / den[:, None]
    ref = ref + torch.from_numpy(value_center).float()[kv_for_query]
    return ref.numpy(), (torch.log2(den) + merged_max).numpy()


@pytest.mark.parametrize("tail_tokens", [1, 15, 16, 17, 241, 255, 256])
def test_exact_tail_merge_center_matches_reference_test_oracle(tail_tokens):
    rng = np.random.default_rng(tail_tokens)
    ring = 18
    exact_key = _f16((ring, 16, 8, 128), 0.35, rng)
    exact_value = _f16((ring, 16, 8, 128), 0.35, rng)
    center = _f16((8, 128), 0.1, rng)
    query = _f16((1, 32, 128), 1.0, rng)
    n = (tail_tokens + 15) // 16
    indices = (np.arange(7, 7 + n) % ring).astype(np.int32)      # wrapped ring addressing
    last = np.array([(tail_tokens - 1) % 16 + 1], np.int32)
    old_output = _f16((1, 32, 128), 0.2, rng)
    old_lse = (rng.standard_normal((1, 32)) * 0.5 + 8.0).astype(np.float32)
    s = 1.0 / math.sqrt(128)
    out, lse = oracle.exact_tail_merge_center(query, exact_key, exact_value, indices, last,
                                              old_output, old_lse, center, s)
    ref, ref_lse = _reference_tail_oracle(query[0], exact_key, exact_value, indices, tail_tokens,
                                          old_output[0], old_lse[0], center, s)
    np.testing.assert_allclose(out[0].astype(np.float32), ref, atol=3e-3, rtol=2e-3)
    np.testing.assert_allclose(lse[0], ref_lse, atol=2e-4, rtol=2e-5)


def test_c_decode_equals_numpy_decode_with_tail_and_center():
    k_codes, v_codes, k_scale, v_scale = _random_paged(30, 9)
    rng = np.random.default_rng(10)
    perm = rng.permutation(30).astype(np.int32)
    indptr = np.array([0, 10, 11, 30], np.int32)
    last = np.array([16, 1, 9], np.int32)
    tail_k, tail_v = _f16((9, 16, 8, 128), 0.3, rng), _f16((9, 16, 8, 128), 0.3, rng)
    tail_indptr = np.array([0, 3, 3, 9], np.int32)
    tail_idx = rng.permutation(9).astype(np.int32)
    tail_last = np.array([4, 16, 16], np.int32)
    q = _f16((3, 32, 128), 1.0, rng)
    center = _f16((3, 8, 128), 0.2, rng)
    s = 1.0 / math.sqrt(128)
    ref = oracle.decode(q, k_codes, v_codes, indptr, perm, last, s, k_scale=k_scale,
                        v_scale=v_scale, tail_k=tail_k, tail_v=tail_v, tail_indptr=tail_indptr,
                        tail_indices=tail_idx, tail_last_page_len=tail_last, value_center=center)
    out, lse = c_oracle.decode_page_gauge(q, k_codes, v_codes, k_scale, v_scale, indptr, perm,
                                          last, s, tail_k, tail_v, tail_indptr, tail_idx,
                                          tail_last, center)
    assert np.abs(out.astype(np.float64) - ref[2]).max() < 2e-3
    np.testing.assert_allclose(lse, ref[1], atol=1e-4)


def test_pinned_table_covers_every_public_function():
    public = {"rope_rotate", "rope_append_fp16", "rope_append_page_gauge", "finalize_codes",
              "quantize_page_gauge", "quantize_completed_kv_pages", "append_finalize_page_gauge",
              "decode", "merge_state", "exact_tail_merge_center"}
    assert public <= set(oracle.PINNED)


# ---------------------------------------------------------------------------
# Sensitivity: plausible mistakes planted in copies of oracle functions (CPU
# only) must be caught by the independent checks above.
# ---------------------------------------------------------------------------

def test_pins_catch_planted_mistakes():
    cos_t, sin_t = oracle.rope_tables(100)
    x = _f16((2, 32, 128), 3.0)
    c, s = cos_t[77], sin_t[77]
    tx, tc, ts = torch.from_numpy(x), torch.from_numpy(c), torch.from_numpy(s)
    reference_rope = (tx * tc + torch.cat((-tx[..., 64:], tx[..., :64]), dim=-1) * ts).numpy()

    # wrong partner sign (the flip on the upper half instead of the lower)
    partner = np.concatenate((x[..., 64:], -x[..., :64]), axis=-1)
    wrong = oracle.f16(oracle.f16(x.astype(np.float64) * c) + oracle.f16(partner.astype(np.float64) * s))
    assert not _bits_equal(wrong, reference_rope)
    # fused multiply-add instead of separately rounded products
    fused = oracle.f16(x.astype(np.float64) * c + np.concatenate((-x[..., 64:], x[..., :64]), -1) * s)
    assert not _bits_equal(fused, reference_rope)

    # half-even instead of half-away rounding of the quotient
    q = (RNG.integers(-100, 100, 500) + 0.5).astype(np.float32)
    half_even = np.clip(np.rint(q), -127, 127).astype(np.int8)
    assert not np.array_equal(half_even, [_sign_symmetric_exact(v) for v in q])

    # scale without the 2^-20 floor, or computed in fp16
    zero = np.zeros((1, 16, 1, 128), np.float32)
    assert np.float16(0.0) != oracle.page_scale(zero, axis=(1, 3))[0, 0]

    # GQA mapping qh % Hkv instead of qh // group
    k_codes, v_codes, k_scale, v_scale = _random_paged(3, 4)
    query = _f16((32, 128))
    keys = k_codes.reshape(-1, 8, 128).astype(np.float64)
    vals = v_codes.reshape(-1, 8, 128).astype(np.float64)
    right = oracle.attention_state(query, keys, vals, 0.088)[0]
    permuted = np.concatenate([query[h::8] for h in range(8)])       # heads regrouped
    wrong_gqa = oracle.attention_state(permuted, keys, vals, 0.088)[0]
    assert np.abs(right - wrong_gqa).max() > 1e-3


# ---------------------------------------------------------------------------
# heterogeneous one-table decode (a unified page table, INT8 then FP16)
# ---------------------------------------------------------------------------

# (old_tokens, total_tokens, ring_pages): the reference's nine CASES,
# diagnostics/benchmark_heterogeneous_fa2_correctness.py:63-73
HETERO_CASES = [(256, 256, 1), (0, 1, 2), (0, 15, 2), (0, 16, 2), (16, 17, 4), (16, 31, 4),
                (16, 32, 4), (144, 176, 4), (144, 191, 4)]


@pytest.mark.parametrize("old_tokens,total_tokens,ring_pages", HETERO_CASES)
def test_heterogeneous_oracle_is_dense_softmax_over_logical_sequence(old_tokens, total_tokens,
                                                                     ring_pages):
    rng = np.random.default_rng(old_tokens * 1000 + total_tokens)
    batch, hkv = 2, 2
    total_pages = -(-total_tokens // 16)
    old_pages = old_tokens // 16
    k_codes = rng.integers(-127, 128, (batch * max(old_pages, 1), 16, hkv, 128)).astype(np.int8)
    v_codes = rng.integers(-127, 128, k_codes.shape).astype(np.int8)
    k_scale = (rng.random((k_codes.shape[0], hkv)) * 0.01 + 0.001).astype(np.float16)
    v_scale = (rng.random((k_codes.shape[0], hkv)) * 0.01 + 0.001).astype(np.float16)
    exact_k = np.full((batch * ring_pages, 16, hkv, 128), np.nan, np.float16)
    exact_v = np.full_like(exact_k, np.nan)
    query = (rng.standard_normal((batch, 4 * hkv, 128)) * 0.35).astype(np.float16)
    center = (rng.standard_normal((batch, hkv, 128)) * 0.025).astype(np.float16)
    indices, logical_k, logical_v = [], [], []
    for r in range(batch):
        ks, vs = [], []
        for page in range(total_pages):
            if page < old_pages:
                pid = r * max(old_pages, 1) + page
                indices.append(pid)
                ks.append(k_codes[pid].astype(np.float64) * k_scale[pid].astype(np.float64)[None, :, None])
                vs.append(v_codes[pid].astype(np.float64) * v_scale[pid].astype(np.float64)[None, :, None])
            else:
                pid = r * ring_pages + page % ring_pages
                exact_k[pid] = rng.standard_normal((16, hkv, 128)) * 0.08
                exact_v[pid] = rng.standard_normal((16, hkv, 128)) * 0.08
                indices.append(pid)
                ks.append(exact_k[pid].astype(np.float64))
                vs.append(exact_v[pid].astype(np.float64))
        logical_k.append(np.concatenate(ks)[:total_tokens])
        logical_v.append(np.concatenate(vs)[:total_tokens])
    last = (total_tokens - 1) % 16 + 1
    indptr = np.arange(batch + 1) * total_pages
    old_len = np.full(batch, old_tokens)
    got16, lse, got = oracle.decode_heterogeneous(query, k_codes, v_codes, k_scale, v_scale,
                                                  exact_k, exact_v, indptr, np.array(indices),
                                                  np.full(batch, last), old_len, 128 ** -0.5,
                                                  value_center=center)
    for r in range(batch):
        for h in range(4 * hkv):
            g = h // 4
            s = logical_k[r][:, g] @ query[r, h].astype(np.float64) / np.sqrt(128)
            p = np.exp(s - s.max())
            p /= p.sum()
            want = p @ logical_v[r][:, g] + center[r, g].astype(np.float64)
            assert np.abs(got[r, h] - want).max() < 1e-9
    assert np.isfinite(got).all() and np.isfinite(lse).all()


# ---------------------------------------------------------------------------
# The torch-CPU restatement timed as the CPU baseline (oracle/cpu_baseline.py)
# ---------------------------------------------------------------------------

def _ragged_int8_case(seed=3):
    rng = np.random.default_rng(seed)
    lengths = [3, 1, 0]                      # history pages per request (one empty)
    tails = [2, 1, 1]
    pool = sum(lengths) + 2
    k = rng.integers(-127, 128, (pool, 16, 2, 128), dtype=np.int8)
    v = rng.integers(-127, 128, (pool, 16, 2, 128), dtype=np.int8)
    ks = (rng.random((pool, 2)) * 1e-2 + 1e-3).astype(np.float16)
    vs = (rng.random((pool, 2)) * 1e-2 + 1e-3).astype(np.float16)
    perm = rng.permutation(pool)[:sum(lengths)].astype(np.int32)
    indptr = np.cumsum([0] + lengths).astype(np.int32)
    ring = sum(tails) + 1
    tk = (rng.standard_normal((ring, 16, 2, 128)) * 0.3).astype(np.float16)
    tv = (rng.standard_normal((ring, 16, 2, 128)) * 0.3).astype(np.float16)
    tail_indptr = np.cumsum([0] + tails).astype(np.int32)
    tail_indices = rng.permutation(ring)[:sum(tails)].astype(np.int32)
    q = (rng.standard_normal((3, 8, 128)) * 0.5).astype(np.float16)
    center = (rng.standard_normal((3, 2, 128)) * 0.05).astype(np.float16)
    return dict(query=q, k_pages=k, v_pages=v, indptr=indptr, indices=perm,
                last_page_len=np.array([16, 16, 16], np.int32), sm_scale=128 ** -0.5,
                k_scale=ks, v_scale=vs, tail_k=tk, tail_v=tv, tail_indptr=tail_indptr,
                tail_indices=tail_indices, tail_last_page_len=np.array([5, 16, 1], np.int32),
                value_center=center)


def test_cpu_baseline_decode_matches_the_oracle():
    import torch

    from oracle import cpu_baseline as cb

    case = _ragged_int8_case()
    want_out, want_lse, _ = oracle.decode(**case)
    as_torch = {k: (torch.from_numpy(v) if isinstance(v, np.ndarray) else v) for k, v in case.items()}
    out, lse = cb.decode_dense(**as_torch)
    assert np.abs(out.numpy().astype(np.float64) - want_out.astype(np.float64)).max() <= 1e-3
    assert np.abs(lse.numpy().astype(np.float64) - want_lse.astype(np.float64)).max() <= 1e-4
    # a plausible mistake (GQA heads regrouped as head-major g*Hkv + kv) is caught
    bad = dict(as_torch, query=as_torch["query"].view(3, 4, 2, 128).transpose(1, 2).reshape(3, 8, 128))
    out_bad, _ = cb.decode_dense(**bad)
    assert np.abs(out_bad.numpy().astype(np.float64) - want_out.astype(np.float64)).max() > 1e-2


def test_cpu_baseline_append_is_bit_exact_with_the_oracle():
    import torch

    from oracle import cpu_baseline as cb

    rng = np.random.default_rng(11)
    batch, hkv, ring, code_pages, sink = 3, 2, 3, 6, 1
    cos_np, sin_np = oracle.rope_tables(code_pages * 16)
    kc = (rng.standard_normal((batch, hkv, 128)) * 0.1).astype(np.float16)
    vc = (rng.standard_normal((batch, hkv, 128)) * 0.1).astype(np.float16)
    shapes = [(batch * ring, 16, hkv, 128)] * 2
    host = [np.zeros(s, np.float16) for s in shapes]
    host += [np.zeros((batch * code_pages, 16, hkv, 128), np.int8) for _ in range(2)]
    host += [np.zeros((batch * code_pages, hkv), np.float16) for _ in range(2)]
    mine = [torch.from_numpy(a.copy()) for a in host]
    rq_host = np.zeros((batch, 8, 128), np.float16)
    rq = torch.zeros(batch, 8, 128, dtype=torch.float16)
    start = np.array([0, 5, 17], np.int32)
    for step in range(40):
        q = (rng.standard_normal((batch, 8, 128))).astype(np.float16)
        k = (rng.standard_normal((batch, hkv, 128))).astype(np.float16)
        v = (rng.standard_normal((batch, hkv, 128))).astype(np.float16)
        pos = start + step
        oracle.rope_append_page_gauge_positions(q, k, v, cos_np, sin_np, pos, kc, vc, rq_host,
                                                *host, sink)
        cb.append_positions(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                            torch.from_numpy(cos_np), torch.from_numpy(sin_np),
                            torch.from_numpy(pos), torch.from_numpy(kc), torch.from_numpy(vc), rq,
                            *mine, sink)
        assert np.array_equal(rq.numpy().view(np.uint16), rq_host.view(np.uint16)), step
    for got, want in zip(mine, host):
        assert np.array_equal(got.numpy().view(np.uint8), want.view(np.uint8))
    assert np.abs(host[5]).max() > 0                      # pages were finalized


def test_cpu_baseline_decoder_step_matches_transformers():
    """One step of the CPU decoder against MistralForCausalLM with the same
    weights, its KV cache holding the reconstruction of the PageGauge cache
    (K = c + s*Z or c + ring) and the new token at the next position."""
    import torch
    from transformers import DynamicCache, MistralConfig, MistralForCausalLM

    from oracle import cpu_baseline as cb

    layers, context, hidden, qh, kvh, inter, vocab = 2, 160, 512, 4, 1, 256, 64
    d = cb.CpuDecoder(layers, context, 9, hidden=hidden, q_heads=qh, kv_heads=kvh,
                      intermediate=inter, vocab=vocab, tail_pages=3, steps=4, std=0.05)
    hf = MistralForCausalLM(MistralConfig(
        vocab_size=vocab, hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
        num_attention_heads=qh, num_key_value_heads=kvh, head_dim=128, rope_theta=1.0e6,
        rms_norm_eps=1e-5, max_position_embeddings=512, tie_word_embeddings=False,
        attn_implementation="eager"))
    qw, kw = qh * 128, kvh * 128
    cache = DynamicCache()
    with torch.no_grad():
        hf.model.embed_tokens.weight.copy_(d.embed)
        hf.lm_head.weight.copy_(d.lm_head)
        for i, (layer, w, c) in enumerate(zip(hf.model.layers, d.layers, d.cache)):
            layer.self_attn.q_proj.weight.copy_(w["qkv"][:qw])
            layer.self_attn.k_proj.weight.copy_(w["qkv"][qw:qw + kw])
            layer.self_attn.v_proj.weight.copy_(w["qkv"][qw + kw:])
            layer.self_attn.o_proj.weight.copy_(w["o"])
            layer.mlp.gate_proj.weight.copy_(w["gate_up"][:inter])
            layer.mlp.up_proj.weight.copy_(w["gate_up"][inter:])
            layer.mlp.down_proj.weight.copy_(w["down"])
            pages = context // 16
            old = pages - d.tail_pages
            keys = torch.cat((c["codes_k"][:old].float() * c["scales_k"][:old].float()[:, None, :, None],
                              c["exact_k"][[p % d.tail_pages for p in range(old, pages)]].float()))
            vals = torch.cat((c["codes_v"][:old].float() * c["scales_v"][:old].float()[:, None, :, None],
                              c["exact_v"][[p % d.tail_pages for p in range(old, pages)]].float()))
            keys = keys.reshape(context, kvh, 128) + c["key_center"].float()
            vals = vals.reshape(context, kvh, 128) + c["value_center"].float()
            cache.update(keys.permute(1, 0, 2)[None].contiguous(),
                         vals.permute(1, 0, 2)[None].contiguous(), i)
    hf.eval()
    token = 17
    with torch.no_grad():
        want = hf(torch.tensor([[token]]), position_ids=torch.tensor([[context]]),
                  past_key_values=cache, use_cache=True).logits[0, -1]
    got = d.step(token, context)
    scale = float(want.abs().max())
    print("cpu decoder step vs transformers", float((got - want).abs().max()), scale)
    assert float((got - want).abs().max()) <= 2e-2 * scale
