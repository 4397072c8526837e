"""GPU parity of the prefill cache population: exact token-mean centers and
the bulk quantizer with exact-ring pages, bit-exact against the oracle.

Cases follow diagnostics/benchmark_backend_exclusive.py:372-506 of the
reference (token-major [T,Hkv,128] sources, per-head centers, a strided K/V
slice of a fused QKV projection, exact tail pages stored centered in FP16)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import assert_bit_equal, cpu

pytestmark = pytest.mark.gpu


def _source(gen, tokens, heads, fused_width=None, outliers=True):
    width = heads * 128 if fused_width is None else fused_width
    base = torch.randn(tokens, width, generator=gen)
    if outliers:
        channels = torch.randperm(heads * 128, generator=gen)[:4]
        base[:, channels] *= 8
    x = base.to(torch.float16)
    return x


@pytest.mark.parametrize("tokens,heads", [(1, 8), (63, 8), (64, 8), (65, 2), (1000, 3),
                                          (16384, 8)])
def test_token_major_centers_bit_exact(cuda, tokens, heads):
    from pagegauge_amd.update import token_major_centers

    print(f"centers tokens={tokens} heads={heads}", flush=True)
    gen = torch.Generator().manual_seed(20260840 + tokens)
    fused = _source(gen, tokens, heads, fused_width=heads * 128 * 3)
    key = fused[:, :heads * 128].view(tokens, heads, 128)
    value = fused[:, 2 * heads * 128:].view(tokens, heads, 128)
    dev = fused.to(cuda)
    dk = dev[:, :heads * 128].view(tokens, heads, 128)
    dv = dev[:, 2 * heads * 128:].view(tokens, heads, 128)
    kc, vc = token_major_centers(dk, dv)
    torch.cuda.synchronize()
    assert_bit_equal(kc, oracle.exact_center(key.numpy()[:, None]), "key center")
    assert_bit_equal(vc, oracle.exact_center(value.numpy()[:, None]), "value center")
    # relation to the reference's float32 mean: equal except near ties
    ref = key.float().mean(dim=0).half()
    differ = (ref.view(torch.int16) != kc.cpu().view(torch.int16))
    assert int(differ.sum()) <= max(2, kc.numel() // 100)


def test_token_major_centers_extremes(cuda):
    from pagegauge_amd.update import token_major_centers

    tokens, heads = 4096, 1
    x = np.zeros((tokens, heads, 128), np.float16)
    x[:, 0, 0] = 65504.0                                 # largest finite: exact int64 sum
    x[:, 0, 1] = np.float16(2.0 ** -24)                  # smallest subnormal
    x[::2, 0, 2] = np.float16(-0.0)
    x[1::2, 0, 2] = np.float16(2.0 ** -14)               # smallest normal
    x[:, 0, 3] = np.where(np.arange(tokens) % 2, 1.0, -1.0).astype(np.float16)
    x[0, 0, 4] = np.float16(1.0)                         # mean 1/4096 exactly
    x[:, 0, 5] = np.float16(-3.0)
    d = torch.from_numpy(x).to(cuda)
    kc, vc = token_major_centers(d, d)
    got = cpu(kc)[0]
    assert got[0] == np.float16(65504.0)
    assert got[1] == np.float16(2.0 ** -24)
    assert got[2] == np.float16(2.0 ** -15)
    assert got[3] == 0 and got[4] == np.float16(1.0 / 4096) and got[5] == np.float16(-3.0)
    assert_bit_equal(kc, oracle.exact_center(x[:, None]), "extremes")
    assert torch.equal(kc, vc)


def test_token_major_centers_errors(cuda):
    from pagegauge_amd.update import token_major_centers

    x = torch.zeros(32, 8, 128, device=cuda, dtype=torch.float16)
    with pytest.raises(ValueError, match="identical"):
        token_major_centers(x, x[:16])
    with pytest.raises(ValueError, match="head dimension must be 128"):
        token_major_centers(x[..., :64], x[..., :64])
    with pytest.raises(ValueError, match="at least"):
        token_major_centers(x, x, workspace=torch.empty(8, device=cuda, dtype=torch.uint8))


def test_prefill_page_gauge_bit_exact_with_exact_ring(cuda):
    from pagegauge_amd.update import prefill_page_gauge, token_major_centers

    gen = torch.Generator().manual_seed(20260841)
    pages, heads, ring_pages = 40, 8, 18
    tokens = pages * 16
    fused = _source(gen, tokens, heads, fused_width=6144)     # q | k | v widths 4096|1024|1024
    key = fused[:, 4096:5120].reshape(pages, 16, heads, 128)
    value = fused[:, 5120:].reshape(pages, 16, heads, 128)
    dev = fused.to(cuda)
    dk = dev[:, 4096:5120].view(tokens, heads, 128)
    dv = dev[:, 5120:].view(tokens, heads, 128)
    kc, vc = token_major_centers(dk, dv)
    codes = [torch.zeros(pages, 16, heads, 128, device=cuda, dtype=torch.int8) for _ in range(2)]
    scales = [torch.zeros(pages, heads, device=cuda, dtype=torch.float16) for _ in range(2)]
    sentinel = np.float16(7.0)
    rings = [torch.full((ring_pages, 16, heads, 128), float(sentinel), device=cuda,
                        dtype=torch.float16) for _ in range(2)]
    exact_map = torch.full((pages,), -1, dtype=torch.int32)
    exact_map[0] = 0                                      # sink slot
    for i, logical in enumerate(range(pages - 16, pages)):
        exact_map[logical] = 2 + (logical % 16)           # tail ring after two fixed slots
    prefill_page_gauge(dk, dv, kc, vc, codes[0], codes[1], scales[0], scales[1],
                       exact_map.to(cuda), rings[0], rings[1])
    torch.cuda.synchronize()
    hk, hv = cpu(kc), cpu(vc)
    want = oracle.quantize_completed_kv_pages(key.numpy(), value.numpy(), hk, hv)
    assert_bit_equal(codes[0], want[0], "key codes")
    assert_bit_equal(codes[1], want[1], "value codes")
    assert_bit_equal(scales[0], want[2], "key scales")
    assert_bit_equal(scales[1], want[3], "value scales")
    ring_k, ring_v = cpu(rings[0]), cpu(rings[1])
    written = set()
    for logical in range(pages):
        slot = int(exact_map[logical])
        if slot < 0:
            continue
        written.add(slot)
        for ring, src, center in ((ring_k, key, hk), (ring_v, value, hv)):
            want_page = oracle.f16(src[logical].numpy().astype(np.float32)
                                   - center.astype(np.float32)[None])
            assert np.array_equal(ring[slot].view(np.uint16), want_page.view(np.uint16)), logical
    for slot in set(range(ring_pages)) - written:
        assert (ring_k[slot] == sentinel).all() and (ring_v[slot] == sentinel).all()


def test_prefill_without_map_equals_bulk_quantizer(cuda):
    from pagegauge_amd.update import prefill_page_gauge, quantize_completed_kv_pages

    gen = torch.Generator().manual_seed(20260842)
    pages, heads = 12, 8
    k = _source(gen, pages * 16, heads).view(pages, 16, heads, 128).to(cuda)
    v = _source(gen, pages * 16, heads).view(pages, 16, heads, 128).to(cuda)
    c = (torch.randn(heads, 128, generator=gen) * 0.1).to(torch.float16).to(cuda)
    out = [torch.empty(pages, 16, heads, 128, device=cuda, dtype=torch.int8) for _ in range(4)]
    sc = [torch.empty(pages, heads, device=cuda, dtype=torch.float16) for _ in range(4)]
    quantize_completed_kv_pages(k, v, c, c, out[0], out[1], sc[0], sc[1])
    prefill_page_gauge(k.view(-1, heads, 128), v.view(-1, heads, 128), c, c, out[2], out[3],
                       sc[2], sc[3])
    torch.cuda.synchronize()
    assert torch.equal(out[0], out[2]) and torch.equal(out[1], out[3])
    assert torch.equal(sc[0], sc[2]) and torch.equal(sc[1], sc[3])
