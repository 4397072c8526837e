"""GPU parity of the fused decoder projection (``pg_decoder_gemv``) against
a float32 PyTorch reference of the same op, and of the fused decoder step
against the torch-op decoder step.

Tolerances: the kernel accumulates in float32 in a different order than the
reference and rounds once to FP16, so outputs agree to one FP16 rounding
(rtol 2^-10) plus float32 accumulation noise; RMSNorm inputs may differ by
one FP16 ulp where rsqrt rounds differently (rtol 2^-9), and a SwiGLU output
compounds the roundings of gate and up (rtol 2^-8)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _rand(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.float16)


def _check(got, want32, rtol):
    diff = (got.float() - want32).abs()
    bound = want32.abs() * rtol + 2e-3
    assert bool((diff <= bound).all()), f"max diff {float(diff.max()):.4g}"


@pytest.mark.parametrize("n,k,batch", [(6144, 4096, 1), (4096, 4096, 2), (1001, 512, 1),
                                       (3, 1024, 4), (32768, 4096, 1)])
def test_projection_plain_and_residual(cuda, n, k, batch):
    from pagegauge_amd.decoder import projection

    print(f"projection n={n} k={k} batch={batch}", flush=True)
    gen = torch.Generator().manual_seed(n + k + batch)
    w = _rand(gen, n, k, scale=0.02).to(cuda)
    x = _rand(gen, batch, k).to(cuda)
    out = torch.empty(batch, n, device=cuda, dtype=torch.float16)
    projection(w, x, out)
    ref = x.float() @ w.float().t()
    _check(out, ref, 2 ** -10)
    res = _rand(gen, batch, n).to(cuda)
    hidden = res.clone()
    projection(w, x, hidden, residual=hidden)              # in place, as the decoder uses it
    want = (res.float() + (x.float() @ w.float().t()).half().float()).half().float()
    _check(hidden, want, 2 ** -9)
    out32 = torch.empty(batch, n, device=cuda, dtype=torch.float32)
    projection(w, x, out32)
    assert torch.equal(out32, out.float())                # FP16 result widened


@pytest.mark.parametrize("k,batch", [(4096, 1), (4096, 2), (512, 3)])
def test_projection_rmsnorm_prologue(cuda, k, batch):
    from pagegauge_amd.decoder import projection, rms_norm

    gen = torch.Generator().manual_seed(k * batch)
    n = 2048
    w = _rand(gen, n, k, scale=0.02).to(cuda)
    x = _rand(gen, batch, k, scale=3.0).to(cuda)
    g = (1.0 + 0.25 * torch.randn(k, generator=gen)).to(torch.float16).to(cuda)
    out = torch.empty(batch, n, device=cuda, dtype=torch.float16)
    projection(w, x, out, norm_weight=g, eps=1e-5)
    ref = rms_norm(x, g, 1e-5).float() @ w.float().t()
    _check(out, ref, 2 ** -9)


@pytest.mark.parametrize("n,k,batch,norm", [(28672, 4096, 1, True), (28672, 4096, 2, True),
                                            (2048, 4096, 1, False), (1024, 512, 4, True)])
def test_projection_swiglu_epilogue(cuda, n, k, batch, norm):
    from pagegauge_amd.decoder import projection, rms_norm

    gen = torch.Generator().manual_seed(n + k + batch)
    w = _rand(gen, n, k, scale=0.02).to(cuda)
    x = _rand(gen, batch, k, scale=2.0).to(cuda)
    g = (1.0 + 0.25 * torch.randn(k, generator=gen)).to(torch.float16).to(cuda)
    out = torch.empty(batch, n // 2, device=cuda, dtype=torch.float16)
    projection(w, x, out, norm_weight=g if norm else None, swiglu=True)
    xin = rms_norm(x, g, 1e-5) if norm else x
    gate, up = (xin.float() @ w.float().t()).half().split(n // 2, dim=-1)
    want = (F.silu(gate) * up).float()                    # FP16 ops as the decoder layer
    _check(out, want, 2 ** -8)


@pytest.mark.parametrize("k,batch", [(14336, 1), (14336, 4), (1024, 2)])
def test_projection_down_with_residual(cuda, k, batch):
    from pagegauge_amd.decoder import projection

    gen = torch.Generator().manual_seed(k + batch)
    n = 4096
    w = _rand(gen, n, k, scale=0.02).to(cuda)
    x = _rand(gen, batch, k).to(cuda)
    res = _rand(gen, batch, n).to(cuda)
    hidden = res.clone()
    projection(w, x, hidden, residual=hidden)
    want = (res.float() + (x.float() @ w.float().t()).half().float()).half().float()
    _check(hidden, want, 2 ** -9)


def test_projection_errors(cuda):
    from pagegauge_amd.decoder import projection

    w = torch.zeros(64, 4096, device=cuda, dtype=torch.float16)
    x = torch.zeros(1, 4096, device=cuda, dtype=torch.float16)
    out = torch.empty(1, 64, device=cuda, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="multiple of 512"):
        projection(torch.zeros(64, 100, device=cuda, dtype=torch.float16),
                   torch.zeros(1, 100, device=cuda, dtype=torch.float16), out)
    with pytest.raises(RuntimeError, match="batch of 1 to 4"):
        projection(w, torch.zeros(5, 4096, device=cuda, dtype=torch.float16),
                   torch.empty(5, 64, device=cuda, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="LDS staging"):
        big = torch.zeros(64, 10240, device=cuda, dtype=torch.float16)
        projection(big, torch.zeros(4, 10240, device=cuda, dtype=torch.float16),
                   torch.empty(4, 64, device=cuda, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="even n"):
        projection(torch.zeros(63, 4096, device=cuda, dtype=torch.float16), x,
                   torch.empty(1, 31, device=cuda, dtype=torch.float16), swiglu=True)
    with pytest.raises(ValueError, match=r"\[B, N\]"):
        projection(w, x, torch.empty(1, 65, device=cuda, dtype=torch.float16))


def test_fused_decoder_step_matches_torch_op_step(cuda):
    """Same weights and cache: fused projections vs torch ops, logits within
    a few FP16 ulps (different accumulation orders only)."""
    from pagegauge_amd import decoder as dec

    cfg = dec.DecoderConfig(layers=2, intermediate=1024, vocab=512)
    weights = dec.DecoderWeights(cfg, seed=3, device=cuda)
    prompt = torch.randint(0, cfg.vocab, (512,), generator=torch.Generator().manual_seed(4))
    first, _, decoders = dec.build_decoders(weights, prompt, 4, backends=("page_gauge",))
    base = decoders["page_gauge"]
    fused = dec.PageGaugeDecoder(weights, base.cache.clone(), "page_gauge", base.max_pages * 16,
                                 base.rope_cos, base.rope_sin, fused=True)
    plain = dec.PageGaugeDecoder(weights, base.cache.clone(), "page_gauge", base.max_pages * 16,
                                 base.rope_cos, base.rope_sin, fused=False)
    token = first
    for i in range(3):
        a = fused.step(token, 512 + i).clone()
        b = plain.step(token, 512 + i)
        scale = float(b.abs().max())
        assert float((a - b).abs().max()) <= 0.02 * max(1.0, scale), i
        assert float(F.cosine_similarity(a, b, dim=-1).min()) > 0.9999
        token = b.argmax(-1)


@pytest.mark.parametrize("centered,batch", [(True, 2), (False, 2), (True, 1)])
def test_qkv_rope_append_is_projection_then_cache_update(cuda, centered, batch):
    """pg_decoder_qkv_rope_append against pg_decoder_gemv followed by the K2
    per-request-positions launch, bit for bit: rotated queries and the ring
    (or FP16 page) rows; row 1 sits past the cache capacity and writes
    nothing.  Positions stay off page ends, where K2 also finalizes."""
    from pagegauge_amd.decoder import projection, qkv_rope_append, rope_tables
    from pagegauge_amd.runtime import load_append_extension

    print(f"qkv append centered={centered} batch={batch}", flush=True)
    ext = load_append_extension()
    gen = torch.Generator().manual_seed(77 + batch + 2 * centered)
    hq, hkv, k, pages, sink = 32, 8, 4096, 6, 1
    w = _rand(gen, (hq + 2 * hkv) * 128, k, scale=0.02).to(cuda)
    x = _rand(gen, batch, k).to(cuda)
    g = _rand(gen, k, scale=0.5).to(cuda)
    cos, sin = (t.to(cuda) for t in rope_tables(pages * 16, 1.0e6))
    positions = torch.tensor([37, 10_000][:batch], dtype=torch.int32, device=cuda)
    kc = _rand(gen, batch, hkv, 128, scale=0.1).to(cuda)
    vc = _rand(gen, batch, hkv, 128, scale=0.1).to(cuda)
    ring = 4 if centered else pages
    shape = (batch * ring, 16, hkv, 128)
    bufs = [dict(q=torch.zeros(batch, hq, 128, device=cuda, dtype=torch.float16),
                 k=torch.zeros(shape, device=cuda, dtype=torch.float16),
                 v=torch.zeros(shape, device=cuda, dtype=torch.float16)) for _ in range(2)]
    fused, ref = bufs
    qkv_rope_append(w, x, norm_weight=g, eps=1e-5, query_heads=hq, kv_heads=hkv, cos=cos, sin=sin,
                    positions=positions, rotated_query=fused["q"], key_pages=fused["k"],
                    value_pages=fused["v"], key_center=kc if centered else None,
                    value_center=vc if centered else None, pages_per_request=ring,
                    sink_pages=sink if centered else 0, capacity_tokens=pages * 16)
    qkv = torch.empty(batch, (hq + 2 * hkv) * 128, device=cuda, dtype=torch.float16)
    projection(w, x, qkv, norm_weight=g, eps=1e-5)
    q = qkv[:, :hq * 128].reshape(batch, hq, 128)
    kk = qkv[:, hq * 128:(hq + hkv) * 128].reshape(batch, hkv, 128)
    vv = qkv[:, (hq + hkv) * 128:].reshape(batch, hkv, 128)
    if centered:
        codes = torch.zeros(batch * pages, 16, hkv, 128, device=cuda, dtype=torch.int8)
        scales = torch.zeros(batch * pages, hkv, device=cuda, dtype=torch.float16)
        ext.rope_append_page_gauge_positions(q.contiguous(), kk.contiguous(), vv.contiguous(),
                                             cos, sin, positions, kc, vc, ref["q"], ref["k"],
                                             ref["v"], codes, codes.clone(), scales,
                                             scales.clone(), sink)
    else:
        for b in range(batch):
            p = int(positions[b])
            if p >= pages * 16:
                continue
            ext.rope_append_fp16_dynamic(q[b:b + 1].contiguous(), kk[b:b + 1].contiguous(),
                                         vv[b:b + 1].contiguous(), cos, sin, positions[b:b + 1],
                                         ref["q"][b:b + 1], ref["k"][b * pages:(b + 1) * pages],
                                         ref["v"][b * pages:(b + 1) * pages])
    torch.cuda.synchronize()
    for name in ("q", "k", "v"):
        assert torch.equal(fused[name], ref[name]), name
    assert fused["k"].abs().sum() > 0
    if batch > 1:
        assert not fused["q"][1].any()              # out-of-capacity row: no writes


def test_qkv_rope_append_rejects_bad_geometry(cuda):
    """Host checks keep every write of the fused cache update inside its
    tensors (the kernel itself trusts them)."""
    from pagegauge_amd.decoder import qkv_rope_append, rope_tables

    hq, hkv, k = 32, 8, 4096
    w = torch.zeros((hq + 2 * hkv) * 128, k, device=cuda, dtype=torch.float16)
    x = torch.zeros(1, k, device=cuda, dtype=torch.float16)
    g = torch.ones(k, device=cuda, dtype=torch.float16)
    cos, sin = (t.to(cuda) for t in rope_tables(64, 1.0e6))
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    rq = torch.empty(1, hq, 128, device=cuda, dtype=torch.float16)
    pages = torch.zeros(4, 16, hkv, 128, device=cuda, dtype=torch.float16)
    kc = torch.zeros(1, hkv, 128, device=cuda, dtype=torch.float16)
    ok = dict(norm_weight=g, eps=1e-5, query_heads=hq, kv_heads=hkv, cos=cos, sin=sin,
              positions=pos, rotated_query=rq, key_pages=pages, value_pages=pages.clone(),
              key_center=kc, value_center=kc.clone(), pages_per_request=4, sink_pages=1,
              capacity_tokens=64)
    qkv_rope_append(w, x, **ok)
    for change, message in ((dict(pages_per_request=5), "pages_per_request"),
                            (dict(sink_pages=4), "tail page"),
                            (dict(key_center=None, value_center=None, capacity_tokens=65),
                             "capacity"),
                            (dict(rotated_query=rq[:, :16]), "rotated_query"),
                            (dict(key_center=kc[:, :4]), "centers"),
                            (dict(positions=torch.zeros(2, dtype=torch.int32, device=cuda)),
                             "positions")):
        with pytest.raises(ValueError, match=message):
            qkv_rope_append(w, x, **{**ok, **change})


@pytest.mark.parametrize("rows,n,stride", [(1, 32768, 32768), (4, 32768, 32768), (3, 1001, 1003),
                                           (2, 5, 8)])
def test_argmax_rows_is_torch_argmax(cuda, rows, n, stride):
    """pg_argmax_f32 against torch.argmax: random rows, a tie planted at two
    positions (the first wins), a NaN (it wins), an all -inf row (index 0),
    rows that are not 16-byte aligned."""
    from pagegauge_amd.decoder import argmax_rows

    print(f"argmax rows={rows} n={n} stride={stride}", flush=True)
    gen = torch.Generator().manual_seed(rows * 7 + n)
    base = torch.randn(rows, stride, generator=gen)
    if rows > 1:
        top = float(base[1, :n].max()) + 1.0
        base[1, n // 3] = top
        base[1, n - 1] = top                      # later tie: the first index wins
    if rows > 2:
        base[2, n // 2] = float("nan")
        base[2, 0] = float("inf")
    x = base.to(cuda)[:, :n]
    if rows == 4:
        x[3] = -float("inf")
    out = torch.empty(rows, device=cuda, dtype=torch.int64)
    argmax_rows(x, out)
    want = torch.argmax(x, dim=-1)
    torch.cuda.synchronize()
    assert torch.equal(out, want), (out.tolist(), want.tolist())
