"""The fused RoPE + centered append + completed-page finalize with head
counts other than 32 query / 8 KV heads (the kernels take both at run
time), bit-exact against the oracle: static and device-position ABIs over
eight pages of tokens with a one-page exact prefix and a two-page ring (so
the ring wraps and every page closes), and the FP16 baseline append."""

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
