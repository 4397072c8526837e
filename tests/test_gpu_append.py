"""GPU parity of the cache-update kernels (bit-exact against the oracle).

Scenarios follow tests/test_page_gauge_append_extension.py of the reference
(static vs device-position ABIs, ring wraps, exact prefix slots, request-major
placement, error messages) and the per-request config-4 update.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import assert_bit_equal, cpu, max_abs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext(cuda):
    from pagegauge_amd import runtime

    return runtime.load_append_extension()


def _rand(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.float16)


def test_rope_append_fp16_static_and_dynamic_bit_exact(ext, cuda):
    # reference test :21-92 (random RoPE tables, 48 positions, ring of 3 pages)
    gen = torch.Generator().manual_seed(20261003)
    batch, pages = 2, 3
    cos, sin = _rand(gen, 48, 128), _rand(gen, 48, 128)
    q = _rand(gen, batch, 32, 128)
    keys, values = _rand(gen, 48, batch, 8, 128), _rand(gen, 48, batch, 8, 128)
    d = lambda t: t.to(cuda)  # noqa: E731
    sq, dq = torch.empty_like(d(q)), torch.empty_like(d(q))
    sk = torch.zeros(batch * pages, 16, 8, 128, dtype=torch.float16, device=cuda)
    sv, dk, dv = torch.zeros_like(sk), torch.zeros_like(sk), torch.zeros_like(sk)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    host = [np.zeros((batch, 32, 128), np.float16), np.zeros(sk.shape, np.float16),
            np.zeros(sk.shape, np.float16)]
    dcos, dsin, dqq = d(cos), d(sin), d(q)
    for p in range(48):
        ext.rope_append_fp16(dqq, d(keys[p]), d(values[p]), dcos[p], dsin[p], sq, sk, sv, p)
        pos.fill_(p)
        ext.rope_append_fp16_dynamic(dqq, d(keys[p]), d(values[p]), dcos, dsin, pos, dq, dk, dv)
        oracle.rope_append_fp16(q.numpy(), keys[p].numpy(), values[p].numpy(), cos[p].numpy(),
                                sin[p].numpy(), *host, p)
    torch.cuda.synchronize()
    assert_bit_equal(sq, host[0], "rotated query")
    assert_bit_equal(sk, host[1], "key pages")
    assert_bit_equal(sv, host[2], "value pages")
    assert torch.equal(sq, dq) and torch.equal(sk, dk) and torch.equal(sv, dv)
    # the reference test's torch formula (fp16 tensor ops)
    expected = q * cos[47] + torch.cat((-q[..., 64:], q[..., :64]), dim=-1) * sin[47]
    assert torch.equal(sq.cpu(), expected)


def _page_gauge_state(batch, ring_pages, code_pages, cuda):
    shapes = [(batch * ring_pages, 16, 8, 128, torch.float16)] * 2 + \
             [(batch * code_pages, 16, 8, 128, torch.int8)] * 2 + \
             [(batch * code_pages, 8, torch.float16)] * 2
    dev = [torch.zeros(s[:-1], dtype=s[-1], device=cuda) for s in shapes]
    host = [cpu(t).copy() for t in dev]
    return dev, host


@pytest.mark.parametrize("sink", [0, 1, 3])
def test_rope_append_page_gauge_static_dynamic_bit_exact(ext, cuda, sink):
    # reference tests :94-161, :282-518 (ring wraps, exact prefix slots)
    gen = torch.Generator().manual_seed(20260821 + sink)
    batch, code_pages, tail_pages = 2, 8, 2
    ring_pages = sink + tail_pages
    n = code_pages * 16
    cos, sin = _rand(gen, n, 128), _rand(gen, n, 128)
    q = _rand(gen, batch, 32, 128)
    keys, values = _rand(gen, n, batch, 8, 128), _rand(gen, n, batch, 8, 128)
    kc, vc = _rand(gen, batch, 8, 128, scale=0.1), _rand(gen, batch, 8, 128, scale=0.1)
    d = lambda t: t.to(cuda)  # noqa: E731
    sdev, host = _page_gauge_state(batch, ring_pages, code_pages, cuda)
    ddev, _ = _page_gauge_state(batch, ring_pages, code_pages, cuda)
    sq, dq = torch.zeros(batch, 32, 128, dtype=torch.float16, device=cuda), None
    dq = torch.zeros_like(sq)
    hq = np.zeros((batch, 32, 128), np.float16)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    dcos, dsin, dqq, dkc, dvc = d(cos), d(sin), d(q), d(kc), d(vc)
    for p in range(n):
        k, v = d(keys[p]), d(values[p])
        ext.rope_append_page_gauge(dqq, k, v, dcos[p], dsin[p], dkc, dvc, sq, *sdev, sink, p)
        pos.fill_(p)
        ext.rope_append_page_gauge_dynamic(dqq, k, v, dcos, dsin, pos, dkc, dvc, dq, *ddev, sink)
        oracle.rope_append_page_gauge(q.numpy(), keys[p].numpy(), values[p].numpy(),
                                      cos[p].numpy(), sin[p].numpy(), kc.numpy(), vc.numpy(), hq,
                                      *host, sink, p)
    torch.cuda.synchronize()
    assert_bit_equal(sq, hq, "rotated query")
    names = ["exact_k", "exact_v", "codes_k", "codes_v", "scales_k", "scales_v"]
    for name, got, dyn, want in zip(names, sdev, ddev, host):
        assert_bit_equal(got, want, name)
        assert torch.equal(got, dyn), name


def test_finalize_reconstruction_and_identity_rope(ext, cuda):
    # reference test :164-215: identity RoPE, one page, rel-L2 < 0.02
    gen = torch.Generator().manual_seed(41)
    q = _rand(gen, 1, 32, 128)
    keys, values = _rand(gen, 16, 1, 8, 128), _rand(gen, 16, 1, 8, 128)
    cos = torch.ones(128, dtype=torch.float16)
    sin = torch.zeros(128, dtype=torch.float16)
    kc, vc = _rand(gen, 8, 128, scale=0.1), _rand(gen, 8, 128, scale=0.1)
    dev, _ = _page_gauge_state(1, 1, 1, cuda)
    rq = torch.empty(1, 32, 128, dtype=torch.float16, device=cuda)
    for p in range(16):
        ext.rope_append_page_gauge(q.to(cuda), keys[p].to(cuda), values[p].to(cuda), cos.to(cuda),
                                   sin.to(cuda), kc.to(cuda), vc.to(cuda), rq, *dev, 0, p)
    torch.cuda.synchronize()
    assert torch.equal(rq.cpu(), q)
    exact_k, _, codes_k, _, scales_k, _ = (t.cpu() for t in dev)
    torch.testing.assert_close(exact_k.float() + kc[None, None].float(),
                               keys[:, 0].float().unsqueeze(0), atol=1.5e-3, rtol=0.0)
    recon = codes_k.float() * scales_k[:, None, :, None].float() + kc[None, None].float()
    ref = keys[:, 0].float().unsqueeze(0)
    assert float((recon - ref).norm() / ref.norm()) < 0.02


def test_positions_variant_config4_bit_exact(ext, cuda):
    # config 4: B=8, 16 steps, 4 rows start unaligned and cross a page boundary
    gen = torch.Generator().manual_seed(20260840)
    start = [4096, 4099, 8192, 8199, 12288, 12299, 16384, 16398]
    batch, ring_pages = 8, 16
    code_pages = (max(start) + 16 + 15) // 16
    cos_np, sin_np = oracle.rope_tables(max(start) + 16)
    cos, sin = torch.from_numpy(cos_np), torch.from_numpy(sin_np)
    kc, vc = _rand(gen, batch, 8, 128, scale=0.1), _rand(gen, batch, 8, 128, scale=0.1)
    dev, host = _page_gauge_state(batch, ring_pages, code_pages, cuda)
    # pre-fill rings with random centered history so finalize reads real rows
    for t_dev, t_host in zip(dev[:2], host[:2]):
        fill = _rand(gen, *t_dev.shape)
        t_dev.copy_(fill.to(cuda))
        t_host[...] = fill.numpy()
    rq = torch.zeros(batch, 32, 128, dtype=torch.float16, device=cuda)
    hq = np.zeros((batch, 32, 128), np.float16)
    dcos, dsin = cos.to(cuda), sin.to(cuda)
    closed = 0
    for step in range(16):
        positions = torch.tensor([s + step for s in start], dtype=torch.int32)
        closed += int(((positions % 16) == 15).sum())
        q = _rand(gen, batch, 32, 128)
        k, v = _rand(gen, batch, 8, 128), _rand(gen, batch, 8, 128)
        ext.rope_append_page_gauge_positions(q.to(cuda), k.to(cuda), v.to(cuda), dcos, dsin,
                                             positions.to(cuda), kc.to(cuda), vc.to(cuda), rq,
                                             *dev, 0)
        oracle.rope_append_page_gauge_positions(q.numpy(), k.numpy(), v.numpy(), cos_np, sin_np,
                                                positions.numpy(), kc.numpy(), vc.numpy(), hq,
                                                *host, 0)
    torch.cuda.synchronize()
    assert closed == 8  # every row closes exactly one page in 16 steps
    assert_bit_equal(rq, hq, "rotated query")
    for name, got, want in zip(["exact_k", "exact_v", "codes_k", "codes_v", "scales_k", "scales_v"],
                               dev, host):
        assert_bit_equal(got, want, name)


def test_positions_variant_equals_scalar_kernel_per_row(ext, cuda):
    gen = torch.Generator().manual_seed(5)
    batch, ring_pages, code_pages = 3, 2, 4
    cos, sin = _rand(gen, 64, 128), _rand(gen, 64, 128)
    positions = [15, 31, 47]
    q = _rand(gen, batch, 32, 128)
    k, v = _rand(gen, batch, 8, 128), _rand(gen, batch, 8, 128)
    kc, vc = _rand(gen, batch, 8, 128, scale=0.1), _rand(gen, batch, 8, 128, scale=0.1)
    ring = _rand(gen, batch * ring_pages, 16, 8, 128)
    multi, _ = _page_gauge_state(batch, ring_pages, code_pages, cuda)
    multi[0].copy_(ring.to(cuda))
    multi[1].copy_(ring.to(cuda))
    rq = torch.zeros(batch, 32, 128, dtype=torch.float16, device=cuda)
    ext.rope_append_page_gauge_positions(q.to(cuda), k.to(cuda), v.to(cuda), cos.to(cuda),
                                         sin.to(cuda), torch.tensor(positions, dtype=torch.int32,
                                                                    device=cuda),
                                         kc.to(cuda), vc.to(cuda), rq, *multi, 0)
    for r, p in enumerate(positions):
        single, _ = _page_gauge_state(1, ring_pages, code_pages, cuda)
        single[0].copy_(ring[r * ring_pages:(r + 1) * ring_pages].to(cuda))
        single[1].copy_(ring[r * ring_pages:(r + 1) * ring_pages].to(cuda))
        srq = torch.zeros(1, 32, 128, dtype=torch.float16, device=cuda)
        ext.rope_append_page_gauge(q[r:r + 1].to(cuda), k[r:r + 1].to(cuda), v[r:r + 1].to(cuda),
                                   cos[p].to(cuda), sin[p].to(cuda), kc[r:r + 1].to(cuda),
                                   vc[r:r + 1].to(cuda), srq, *single, 0, p)
        torch.cuda.synchronize()
        assert torch.equal(srq[0], rq[r])
        assert torch.equal(single[0], multi[0][r * ring_pages:(r + 1) * ring_pages])
        assert torch.equal(single[2], multi[2][r * code_pages:(r + 1) * code_pages])
        assert torch.equal(single[4], multi[4][r * code_pages:(r + 1) * code_pages])


def test_error_messages_match_reference(ext, cuda):
    # reference test :520-585
    batch, code_pages, tail_pages, prefix = 2, 8, 2, 3
    q = torch.zeros(batch, 32, 128, dtype=torch.float16, device=cuda)
    k = torch.zeros(batch, 8, 128, dtype=torch.float16, device=cuda)
    cos = torch.ones(4, 128, dtype=torch.float16, device=cuda)
    sin = torch.zeros_like(cos)
    kc = torch.zeros(batch, 8, 128, dtype=torch.float16, device=cuda)
    dev, _ = _page_gauge_state(batch, prefix + tail_pages, code_pages, cuda)
    rq = torch.zeros_like(q)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    with pytest.raises(RuntimeError, match="must be nonnegative"):
        ext.rope_append_page_gauge(q, k, k, cos[0], sin[0], kc, kc, rq, *dev, -1, 0)
    with pytest.raises(RuntimeError, match="at least one tail-ring page"):
        ext.rope_append_page_gauge_dynamic(q, k, k, cos, sin, pos, kc, kc, rq, *dev,
                                           prefix + tail_pages)
    big_k = torch.zeros(batch * (code_pages + tail_pages), 16, 8, 128, dtype=torch.float16,
                        device=cuda)
    with pytest.raises(RuntimeError, match="logical cache capacity"):
        ext.rope_append_page_gauge(q, k, k, cos[0], sin[0], kc, kc, rq, big_k, big_k.clone(),
                                   *dev[2:], code_pages, 0)
    with pytest.raises(RuntimeError, match="position must be non-negative"):
        ext.rope_append_fp16(q, k, k, cos[0], sin[0], rq, big_k, big_k.clone(), -1)


def test_out_of_range_device_position_is_a_noop(ext, cuda):
    batch = 1
    q = torch.randn(batch, 32, 128, device=cuda).half()
    k = torch.randn(batch, 8, 128, device=cuda).half()
    cos = torch.randn(4, 128, device=cuda).half()
    sin = torch.randn(4, 128, device=cuda).half()
    kc = torch.zeros(8, 128, dtype=torch.float16, device=cuda)
    dev, _ = _page_gauge_state(batch, 2, 2, cuda)
    before = [t.clone() for t in dev]
    rq = torch.zeros_like(q)
    for bad in (-1, 4, 31, 32):   # negative, beyond RoPE rows, beyond capacity
        pos = torch.tensor([bad], dtype=torch.int32, device=cuda)
        ext.rope_append_page_gauge_dynamic(q, k, k, cos, sin, pos, kc, kc, rq, *dev, 0)
    torch.cuda.synchronize()
    assert not bool(rq.abs().sum())
    for a, b in zip(dev, before):
        assert torch.equal(a, b)


@pytest.mark.parametrize("tail_tokens", [1, 15, 16, 17, 241, 255, 256])
def test_exact_tail_merge_center_matches_oracle(ext, cuda, tail_tokens):
    # reference test :588-676 (wrapped, non-monotonic ring addressing)
    gen = torch.Generator().manual_seed(97)
    ring_pages = 16
    q = _rand(gen, 1, 32, 128)
    exact_k = _rand(gen, ring_pages, 16, 8, 128, scale=0.35)
    exact_v = _rand(gen, ring_pages, 16, 8, 128, scale=0.35)
    center = _rand(gen, 8, 128, scale=0.1)
    pages = (tail_tokens + 15) // 16
    indices = (torch.arange(7, 7 + pages) % ring_pages).to(torch.int32)
    last = torch.tensor([(tail_tokens - 1) % 16 + 1], dtype=torch.int32)
    old_out = _rand(gen, 1, 32, 128, scale=0.2)
    old_lse = (torch.randn(1, 32, generator=gen) * 0.5 + 8.0).float()
    want_out, want_lse = oracle.exact_tail_merge_center(
        q.numpy(), exact_k.numpy(), exact_v.numpy(), indices.numpy(), last.numpy(),
        old_out.numpy(), old_lse.numpy(), center.numpy(), 128 ** -0.5)
    dout, dlse = old_out.to(cuda), old_lse.to(cuda)
    ext.exact_tail_merge_center(q.to(cuda), exact_k.to(cuda), exact_v.to(cuda), indices.to(cuda),
                                last.to(cuda), dout, dlse, center.to(cuda), 128 ** -0.5)
    torch.cuda.synchronize()
    assert max_abs(dout, want_out) <= 2e-3
    assert max_abs(dlse, want_lse) <= 2e-4


def test_batched_exact_tail_merge_center_ragged(ext, cuda):
    # reference test :832-930: ragged tails [33, 37, 47]
    gen = torch.Generator().manual_seed(173)
    batch, ring_pages, tails = 3, 4, [33, 37, 47]
    q = _rand(gen, batch, 32, 128)
    exact_k = _rand(gen, batch * ring_pages, 16, 8, 128, scale=0.35)
    exact_v = _rand(gen, batch * ring_pages, 16, 8, 128, scale=0.35)
    center = _rand(gen, batch, 8, 128, scale=0.1)
    indices = torch.stack([r * ring_pages + torch.tensor([2, 3, 0]) for r in range(batch)]).reshape(-1)
    indices = indices.to(torch.int32)
    last = torch.tensor([(t - 1) % 16 + 1 for t in tails], dtype=torch.int32)
    old_out = _rand(gen, batch, 32, 128, scale=0.2)
    old_lse = (torch.randn(batch, 32, generator=gen) * 0.5 + 8.0).float()
    want_out, want_lse = oracle.exact_tail_merge_center(
        q.numpy(), exact_k.numpy(), exact_v.numpy(), indices.numpy(), last.numpy(),
        old_out.numpy(), old_lse.numpy(), center.numpy(), 128 ** -0.5)
    dout, dlse = old_out.to(cuda), old_lse.to(cuda)
    ext.exact_tail_merge_center(q.to(cuda), exact_k.to(cuda), exact_v.to(cuda), indices.to(cuda),
                                last.to(cuda), dout, dlse, center.to(cuda), 128 ** -0.5)
    torch.cuda.synchronize()
    assert max_abs(dout, want_out) <= 2e-3
    assert max_abs(dlse, want_lse) <= 2e-4


def test_bulk_quantizer_bit_exact(cuda):
    from pagegauge_amd import workloads

    gen = torch.Generator().manual_seed(21)
    pages, heads = 37, 2
    key, value = _rand(gen, pages, 16, heads, 128), _rand(gen, pages, 16, heads, 128, scale=3.0)
    key[3] = 0  # all-zero page -> scale floor 2^-20
    kc, vc = _rand(gen, heads, 128, scale=0.1), _rand(gen, heads, 128, scale=0.1)
    outs = [torch.empty(pages, 16, heads, 128, dtype=torch.int8, device=cuda) for _ in range(2)]
    outs += [torch.empty(pages, heads, dtype=torch.float16, device=cuda) for _ in range(2)]
    workloads.quantize_completed_kv_pages(key.to(cuda), value.to(cuda), kc.to(cuda), vc.to(cuda),
                                          *outs)
    torch.cuda.synchronize()
    want = oracle.quantize_completed_kv_pages(key.numpy(), value.numpy(), kc.numpy(), vc.numpy())
    for name, got, ref in zip(["key_codes", "value_codes", "key_scales", "value_scales"], outs, want):
        assert_bit_equal(got, ref, name)


def test_paged_append_and_finalize_bit_exact(cuda):
    from pagegauge_amd import update

    gen = torch.Generator().manual_seed(31)
    batch, heads = 3, 2
    inc_k, inc_v = _rand(gen, 16, batch, heads, 128), _rand(gen, 16, batch, heads, 128)
    kc, vc = _rand(gen, heads, 128, scale=0.1), _rand(gen, heads, 128, scale=0.1)
    page_ids = torch.tensor([2, 0, 1], dtype=torch.int32)
    shape = (batch, 16, heads, 128)
    base = [torch.zeros(shape, dtype=torch.float16, device=cuda) for _ in range(2)]
    state = [torch.zeros(shape, dtype=torch.float16, device=cuda) for _ in range(2)]
    state += [torch.zeros(shape, dtype=torch.int8, device=cuda) for _ in range(2)]
    state += [torch.zeros(batch, heads, dtype=torch.float16, device=cuda) for _ in range(2)]
    host_base = [np.zeros(shape, np.float16) for _ in range(2)]
    host = [cpu(t).copy() for t in state]
    dids = page_ids.to(cuda)
    for token in range(16):
        offsets = torch.full((batch,), token, dtype=torch.int32)
        update.append_kv(inc_k[token].to(cuda), inc_v[token].to(cuda), *base, dids,
                         offsets.to(cuda))
        update.append_finalize_page_gauge(inc_k[token].to(cuda), inc_v[token].to(cuda),
                                          kc.to(cuda), vc.to(cuda), *state, dids, offsets.to(cuda))
        oracle.append_kv(inc_k[token].numpy(), inc_v[token].numpy(), *host_base, page_ids.numpy(),
                         offsets.numpy())
        oracle.append_finalize_page_gauge(inc_k[token].numpy(), inc_v[token].numpy(), kc.numpy(),
                                          vc.numpy(), *host, page_ids.numpy(), offsets.numpy())
    torch.cuda.synchronize()
    for got, want in zip(base, host_base):
        assert_bit_equal(got, want, "append_kv")
    for name, got, want in zip(["exact_k", "exact_v", "codes_k", "codes_v", "scales_k", "scales_v"],
                               state, host):
        assert_bit_equal(got, want, name)


def test_page_gauge_quantizer_bit_exact(cuda):
    """a13: the K1 driver's quantize_page_gauge on the GPU (round-half-even
    codes of the float32-centered values), bit-exact against the oracle given
    the center, and the center equal to the oracle's exact mean.  Page 0 holds
    exact half-way quotients (k + 1/2 with scale 1/8), where half-even and the
    finalize's sign-symmetric rounding disagree for even k; page 1 is all zero
    (the 2^-20 scale floor)."""
    from pagegauge_amd import update

    gen = torch.Generator().manual_seed(20260814)
    pages, heads = 41, 8
    values = _rand(gen, pages, 16, heads, 128, scale=2.0)
    ladder = (torch.arange(16 * 128, dtype=torch.float32).reshape(16, 128) % 127 + 0.5) / 8
    ladder[0, 0] = 127 / 8                     # page max: scale = 127/8 / 127 = 1/8 exactly
    sign = torch.where(torch.arange(128) % 2 == 0, 1.0, -1.0)
    values[0] = (ladder * sign).half()[:, None, :].expand(16, heads, 128)
    values[1] = 0
    zero = torch.zeros(heads, 128, dtype=torch.float16)
    codes, center, scale, recon, centered = update.quantize_page_gauge(values.to(cuda), zero.to(cuda))
    torch.cuda.synchronize()
    want = oracle.quantize_page_gauge(values.numpy(), zero.numpy())
    for name, got, ref in zip(["codes", "center", "scale", "reconstructed", "centered"],
                              (codes, center, scale, recon, centered), want):
        assert_bit_equal(got, ref, name)
    assert float(scale[0, 0]) == 0.125
    ties = cpu(codes)[0, :, 0, :].astype(np.int32)
    half_away = np.sign(ladder.numpy() * sign.numpy()) * np.floor(np.abs(ladder.numpy() * 8 * sign.numpy()) + 0.5)
    assert (ties != half_away).any()            # the tie page does tell the two roundings apart
    # the center computed on the GPU (exact token mean) as the reference's center
    codes2, center2, scale2, _, _ = update.quantize_page_gauge(values.to(cuda))
    torch.cuda.synchronize()
    want2 = oracle.quantize_page_gauge(values.numpy())
    assert_bit_equal(center2, want2[1], "center")
    assert_bit_equal(codes2, want2[0], "codes")
    assert_bit_equal(scale2, want2[2], "scale")
