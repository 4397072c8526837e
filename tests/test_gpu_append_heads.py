"""The cache-update kernels with head counts other than 32 query / 8 KV
heads (the kernels take both at run time): the fused RoPE + centered append
+ completed-page finalize, bit-exact against the oracle through the static
and device-position ABIs over eight pages of tokens with a one-page exact
prefix and a two-page ring (so the ring wraps and every page closes); the
FP16 baseline append, bit-exact; and the fused exact-tail merge (GQA group
4) within the reference test's tolerances."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import assert_bit_equal, cpu

pytestmark = pytest.mark.gpu

HEADS = [(4, 1), (8, 2), (16, 4), (64, 16)]


@pytest.fixture(scope="module")
def ext(cuda):
    from pagegauge_amd import runtime

    return runtime.load_append_extension()


def _rand(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.float16)


@pytest.mark.parametrize("hq,hkv", HEADS)
def test_rope_append_page_gauge_any_head_count(ext, cuda, hq, hkv):
    gen = torch.Generator().manual_seed(20260870 + hkv)
    batch, code_pages, tail_pages, sink = 2, 8, 2, 1
    ring_pages = sink + tail_pages
    n = code_pages * 16
    cos, sin = _rand(gen, n, 128), _rand(gen, n, 128)
    q = _rand(gen, batch, hq, 128)
    keys, values = _rand(gen, n, batch, hkv, 128), _rand(gen, n, batch, hkv, 128)
    kc, vc = _rand(gen, batch, hkv, 128, scale=0.1), _rand(gen, batch, hkv, 128, scale=0.1)
    shapes = [(batch * ring_pages, 16, hkv, 128, torch.float16)] * 2 + \
             [(batch * code_pages, 16, hkv, 128, torch.int8)] * 2 + \
             [(batch * code_pages, hkv, torch.float16)] * 2
    sdev = [torch.zeros(s[:-1], dtype=s[-1], device=cuda) for s in shapes]
    ddev = [torch.zeros_like(t) for t in sdev]
    host = [cpu(t).copy() for t in sdev]
    sq = torch.zeros(batch, hq, 128, dtype=torch.float16, device=cuda)
    dq = torch.zeros_like(sq)
    hq_host = np.zeros((batch, hq, 128), np.float16)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    d = lambda t: t.to(cuda)  # noqa: E731
    dcos, dsin, dqq, dkc, dvc = d(cos), d(sin), d(q), d(kc), d(vc)
    for p in range(n):
        k, v = d(keys[p]), d(values[p])
        ext.rope_append_page_gauge(dqq, k, v, dcos[p], dsin[p], dkc, dvc, sq, *sdev, sink, p)
        pos.fill_(p)
        ext.rope_append_page_gauge_dynamic(dqq, k, v, dcos, dsin, pos, dkc, dvc, dq, *ddev, sink)
        oracle.rope_append_page_gauge(q.numpy(), keys[p].numpy(), values[p].numpy(),
                                      cos[p].numpy(), sin[p].numpy(), kc.numpy(), vc.numpy(),
                                      hq_host, *host, sink, p)
    torch.cuda.synchronize()
    assert_bit_equal(sq, hq_host, "rotated query")
    names = ["exact_k", "exact_v", "codes_k", "codes_v", "scales_k", "scales_v"]
    for name, got, dyn, want in zip(names, sdev, ddev, host):
        assert_bit_equal(got, want, name)
        assert torch.equal(got, dyn), name
    assert bool((sdev[4] != 0).all())                  # every page of every request closed


@pytest.mark.parametrize("hq,hkv", HEADS)
def test_rope_append_fp16_any_head_count(ext, cuda, hq, hkv):
    gen = torch.Generator().manual_seed(20260880 + hkv)
    batch, pages = 2, 3
    cos, sin = _rand(gen, 48, 128), _rand(gen, 48, 128)
    q = _rand(gen, batch, hq, 128)
    keys, values = _rand(gen, 48, batch, hkv, 128), _rand(gen, 48, batch, hkv, 128)
    d = lambda t: t.to(cuda)  # noqa: E731
    sq = torch.empty(batch, hq, 128, dtype=torch.float16, device=cuda)
    sk = torch.zeros(batch * pages, 16, hkv, 128, dtype=torch.float16, device=cuda)
    sv = torch.zeros_like(sk)
    host = [np.zeros((batch, hq, 128), np.float16), np.zeros(sk.shape, np.float16),
            np.zeros(sk.shape, np.float16)]
    dcos, dsin, dqq = d(cos), d(sin), d(q)
    for p in range(48):
        ext.rope_append_fp16(dqq, d(keys[p]), d(values[p]), dcos[p], dsin[p], sq, sk, sv, p)
        oracle.rope_append_fp16(q.numpy(), keys[p].numpy(), values[p].numpy(), cos[p].numpy(),
                                sin[p].numpy(), *host, p)
    torch.cuda.synchronize()
    assert_bit_equal(sq, host[0], "rotated query")
    assert_bit_equal(sk, host[1], "key pages")
    assert_bit_equal(sv, host[2], "value pages")


@pytest.mark.parametrize("hq,hkv", HEADS)
def test_exact_tail_merge_center_any_head_count(ext, cuda, hq, hkv):
    from tests.helpers import max_abs

    gen = torch.Generator().manual_seed(20260890 + hkv)
    batch, ring_pages, tails = 2, 8, [117, 113]        # 8 ring pages each, ragged last page
    q = _rand(gen, batch, hq, 128)
    exact_k = _rand(gen, batch * ring_pages, 16, hkv, 128, scale=0.35)
    exact_v = _rand(gen, batch * ring_pages, 16, hkv, 128, scale=0.35)
    center = _rand(gen, batch, hkv, 128, scale=0.1)
    pages = (max(tails) + 15) // 16
    # every request names its 8 ring slots starting mid-ring
    indices = torch.stack([r * ring_pages + (torch.arange(pages) + 5) % ring_pages
                           for r in range(batch)]).reshape(-1).to(torch.int32)
    last = torch.tensor([(t - 1) % 16 + 1 for t in tails], dtype=torch.int32)
    old_out = _rand(gen, batch, hq, 128, scale=0.2)
    old_lse = (torch.randn(batch, hq, generator=gen) * 0.5 + 8.0).float()
    want_out, want_lse = oracle.exact_tail_merge_center(
        q.numpy(), exact_k.numpy(), exact_v.numpy(), indices.numpy(), last.numpy(),
        old_out.numpy(), old_lse.numpy(), center.numpy(), 128 ** -0.5)
    dout, dlse = old_out.to(cuda), old_lse.to(cuda)
    ext.exact_tail_merge_center(q.to(cuda), exact_k.to(cuda), exact_v.to(cuda), indices.to(cuda),
                                last.to(cuda), dout, dlse, center.to(cuda), 128 ** -0.5)
    torch.cuda.synchronize()
    assert max_abs(dout, want_out) <= 2e-3
    assert max_abs(dlse, want_lse) <= 2e-4
