"""Config 1 end to end: prefill + K2 (RoPE theta 1e6) + K1, against the oracle.

B=1, Mistral-7B layer shape, q/K/V ~ N(0,1) fp16 from
seed 20260840, RoPE theta 1e6, 4096 tokens = 240 INT8 pages + a 16-page FP16
exact ring, one decode query.  Following the decoder's step
(scripts/benchmark_page_gauge_transformer.py:3159-3274 -> plan(position+1)):
the first 4080 tokens (255 whole pages) are the prefill (HF-rounded RoPE,
exact token-mean centers, every page quantised, the last 16 prefill pages
copied into the ring), then K2 (``rope_append_page_gauge``) appends the tokens
at positions 4080..4095, which fills page 255 and finalizes it, and the query
of position 4095 (rotated by the last K2 call) attends to the whole context:
INT8 pages 0..239 and ring pages for logical pages 240..255.

Bar: every cache byte (codes, scales, centers, ring) and the rotated query
bit-exact against the same steps on the oracle; the decode output and base-2
LSE within 2e-3 of the oracle's float64 decode of those caches.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import assert_bit_equal, cpu, max_abs

pytestmark = pytest.mark.gpu

SEED = 20260840
TOKENS = 4096
PREFILL = 4080
RING = 16
HKV, HQ, DIM, PAGE = 8, 32, 128, 16


def test_config1_prefill_append_decode_end_to_end(cuda):
    from pagegauge_amd import decode, decoder, runtime

    gen = torch.Generator().manual_seed(SEED)
    q = torch.randn(TOKENS, HQ, DIM, generator=gen).half()
    k = torch.randn(TOKENS, HKV, DIM, generator=gen).half()
    v = torch.randn(TOKENS, HKV, DIM, generator=gen).half()
    cos, sin = decoder.rope_tables(TOKENS, 1.0e6)
    pages = TOKENS // PAGE

    # ---- GPU: prefill, K2 for the last page, K1
    cfg = decoder.DecoderConfig(layers=1, intermediate=512, vocab=1024)
    cache = decoder.GaugeCache(cfg, 1, pages, RING, device=cuda)
    rk = decoder.rope(k[:PREFILL].to(cuda), cos[:PREFILL].to(cuda), sin[:PREFILL].to(cuda))
    cache.populate(0, 0, rk, v[:PREFILL].to(cuda))
    ext = runtime.load_append_extension()
    rotated_q = torch.empty(1, HQ, DIM, dtype=torch.float16, device=cuda)
    for position in range(PREFILL, TOKENS):
        ext.rope_append_page_gauge(
            q[position:position + 1].to(cuda), k[position:position + 1].to(cuda),
            v[position:position + 1].to(cuda), cos[position].to(cuda), sin[position].to(cuda),
            cache.key_center[0], cache.value_center[0], rotated_q, cache.exact_key[0],
            cache.exact_value[0], cache.key_codes[0], cache.value_codes[0], cache.key_scales[0],
            cache.value_scales[0], 0, position)
    old_pages = pages - RING
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=cuda)  # noqa: E731
    old_indptr, old_indices = i32([0, old_pages]), i32(list(range(old_pages)))
    tail_indptr, tail_indices = i32([0, RING]), i32([p % RING for p in range(old_pages, pages)])
    full = i32([PAGE])
    dec = decode.PageGaugeSegmentedDecode(torch.empty(16 << 20, dtype=torch.uint8, device=cuda))
    dec.plan(old_indptr, old_indices, full, tail_indptr, tail_indices, full)
    out, lse = dec.run(rotated_q, (cache.key_codes[0], cache.value_codes[0]), cache.key_scales[0],
                       cache.value_scales[0], (cache.exact_key[0], cache.exact_value[0]),
                       cache.value_center[0], return_lse=True)
    torch.cuda.synchronize()

    # ---- oracle: the same steps
    qn, kn, vn = q.numpy(), k.numpy(), v.numpy()
    cn, sn = cos.numpy(), sin.numpy()
    rk_ref = oracle.rope_rotate(kn[:PREFILL], cn[:PREFILL, None, :], sn[:PREFILL, None, :])
    assert_bit_equal(rk, rk_ref, "prefill RoPE")
    pk = rk_ref.reshape(PREFILL // PAGE, PAGE, HKV, DIM)
    pv = vn[:PREFILL].reshape(PREFILL // PAGE, PAGE, HKV, DIM)
    kc, vc = oracle.exact_center(pk), oracle.exact_center(pv)
    codes_k = np.zeros((pages, PAGE, HKV, DIM), np.int8)
    codes_v = np.zeros_like(codes_k)
    scales_k = np.zeros((pages, HKV), np.float16)
    scales_v = np.zeros_like(scales_k)
    ck, cv, sk, sv = oracle.quantize_completed_kv_pages(pk, pv, kc, vc)
    n_pre = PREFILL // PAGE
    codes_k[:n_pre], codes_v[:n_pre], scales_k[:n_pre], scales_v[:n_pre] = ck, cv, sk, sv
    ring_k = np.zeros((RING, PAGE, HKV, DIM), np.float16)
    ring_v = np.zeros_like(ring_k)
    for page in range(n_pre - RING, n_pre):
        ring_k[page % RING] = oracle.f16(oracle.f32(pk[page]) - oracle.f32(kc))
        ring_v[page % RING] = oracle.f16(oracle.f32(pv[page]) - oracle.f32(vc))
    rq_ref = np.zeros((1, HQ, DIM), np.float16)
    for position in range(PREFILL, TOKENS):
        oracle.rope_append_page_gauge(qn[position:position + 1], kn[position:position + 1],
                                      vn[position:position + 1], cn[position], sn[position],
                                      kc, vc, rq_ref, ring_k, ring_v, codes_k, codes_v,
                                      scales_k, scales_v, 0, position)
    for name, got, want in (("key center", cache.key_center[0, 0], kc),
                            ("value center", cache.value_center[0, 0], vc),
                            ("key codes", cache.key_codes[0], codes_k),
                            ("value codes", cache.value_codes[0], codes_v),
                            ("key scales", cache.key_scales[0], scales_k),
                            ("value scales", cache.value_scales[0], scales_v),
                            ("ring keys", cache.exact_key[0], ring_k),
                            ("ring values", cache.exact_value[0], ring_v),
                            ("rotated query", rotated_q, rq_ref)):
        assert_bit_equal(got, want, name)
    ref_out, ref_lse, _ = oracle.decode(
        rq_ref, codes_k, codes_v, cpu(old_indptr), cpu(old_indices), cpu(full), 128 ** -0.5,
        k_scale=scales_k, v_scale=scales_v, tail_k=ring_k, tail_v=ring_v,
        tail_indptr=cpu(tail_indptr), tail_indices=cpu(tail_indices), tail_last_page_len=cpu(full),
        value_center=vc[None])
    print("config1 e2e", max_abs(out, ref_out), max_abs(lse, ref_lse), flush=True)
    assert max_abs(out, ref_out) <= 2e-3
    assert max_abs(lse, ref_lse) <= 2e-3
