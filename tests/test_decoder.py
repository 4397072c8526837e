"""Host logic of the PageGauge decoder (CPU): the plan guard, the decoder's
page partition, and the model arithmetic pinned against ``transformers``'
Mistral implementation (the library the reference builds its model from).

Golden lists follow tests/test_page_gauge_transformer.py:218-330 of the
reference (``GraphDecodeWrapper`` plan counts and the sink-prefix decoder
plan)."""

from __future__ import annotations

import math

import pytest
import torch

from pagegauge_amd import decoder as dec
from pagegauge_amd import page_table as pt

PAGE = 16


def test_segment_table_replans_only_on_structural_change():
    # reference :218-273 (FlashInfer's plan also keys ceil(tokens/32); the
    # split scheduler here depends on page counts only)
    table = dec.SegmentTable(2, 4, device="cpu")
    indices = torch.tensor([[0, 1], [4, 5]], dtype=torch.int32)
    assert table.plan(indices, logical_tokens=19, last_page_len=3, split_pages=0)
    assert table.indptr.tolist() == [0, 2, 4]
    assert table.active_indices().tolist() == [0, 1, 4, 5]
    assert table.last_len.tolist() == [3, 3]
    assert not table.plan(indices, logical_tokens=20, last_page_len=4, split_pages=0)
    assert table.last_len.tolist() == [4, 4]
    assert table.operation_counts() == {"plan_invocations": 2, "plan_rebuilds": 1,
                                        "last_page_len_device_fills": 2}
    indices[0, 0] = 7
    assert table.plan(indices, logical_tokens=20, last_page_len=4, split_pages=0,
                      page_table_epoch=2)
    assert table.active_indices().tolist() == [7, 1, 4, 5]
    assert table.operation_counts()["plan_rebuilds"] == 2
    # a new split size is a new structure too
    assert table.plan(indices, 20, 4, split_pages=8, page_table_epoch=2)


@pytest.mark.parametrize("kwargs,message", [
    (dict(physical_indices=torch.zeros(3, 2, dtype=torch.int32)), r"shape \[B,pages\]"),
    (dict(physical_indices=torch.zeros(2, 0, dtype=torch.int32)), "at least one page"),
    (dict(logical_tokens=40), "logical tokens do not match"),
    (dict(last_page_len=17), "logical tokens do not match"),
    (dict(physical_indices=torch.zeros(2, 5, dtype=torch.int32), logical_tokens=80,
          last_page_len=16), "exceeds the allocated page table"),
])
def test_segment_table_rejects_bad_plans(kwargs, message):
    table = dec.SegmentTable(2, 4, device="cpu")
    args = dict(physical_indices=torch.zeros(2, 2, dtype=torch.int32), logical_tokens=19,
                last_page_len=3, split_pages=0)
    args.update(kwargs)
    with pytest.raises(ValueError, match=message):
        table.plan(**args)


class _FakeSegmented:
    def __init__(self):
        self.calls = []

    def plan(self, old_indptr, old_indices, old_last, tail_indptr, tail_indices, tail_last,
             *args, **kwargs):
        self.calls.append((old_indptr.tolist(), old_indices.tolist(), old_last.tolist(),
                           tail_indptr.tolist(), tail_indices.tolist(), tail_last.tolist()))


def _plan_only_decoder(batch, max_pages, tail_pages, sink_pages, suffix_pages=0, initial=None):
    d = dec.PageGaugeDecoder.__new__(dec.PageGaugeDecoder)
    d.backend = "page_gauge"
    d.tail_attention = "segmented"
    d.config = dec.DecoderConfig(layers=1, intermediate=8, vocab=8)
    d.decoder_plan_calls = d.kernel_replans = d.exact_page_table_updates = 0
    d.max_pages, d.batch_size = max_pages, batch
    d.exact_tail_pages, d.exact_sink_pages, d.split_pages = tail_pages, sink_pages, 0
    d.exact_static_suffix_pages, d.initial_context_pages = suffix_pages, initial
    d.exact_fixed_pages = sink_pages + suffix_pages
    slots = tail_pages + sink_pages + suffix_pages
    d.all_pages = pt.request_major_page_table(batch, max_pages, device="cpu")
    d.exact_ring_pages = pt.request_major_exact_page_table(batch, max_pages, tail_pages,
                                                           sink_pages, suffix_pages, initial,
                                                           device="cpu")
    d.exact_plan_pages = torch.empty(batch, slots, dtype=torch.int32)
    d.old_plan_pages = torch.empty_like(d.all_pages) if suffix_pages else None
    d.old_layout_signature = None
    d.old_page_table_updates = 0
    d.exact_layout_signature = None
    d.old_table = dec.SegmentTable(batch, max_pages, "cpu")
    d.exact_table = dec.SegmentTable(batch, slots, "cpu")
    d.decode = _FakeSegmented()
    return d


def test_decoder_plan_excludes_sink_from_old_and_prepends_it_to_exact():
    # reference :276-330
    d = _plan_only_decoder(batch=2, max_pages=8, tail_pages=2, sink_pages=1)
    d.plan(8 * PAGE)
    old_indptr, old_indices, old_last, tail_indptr, exact_indices, exact_last = d.decode.calls[-1]
    assert old_indptr == [0, 5, 10]
    assert old_indices == [1, 2, 3, 4, 5, 9, 10, 11, 12, 13]
    assert tail_indptr == [0, 3, 6]
    assert exact_indices == [0, 1, 2, 3, 4, 5]
    assert old_last == [16, 16] and exact_last == [16, 16]
    assert d.old_pages * PAGE == 5 * PAGE and d.exact_pages == 3
    assert d.exact_table.signature[-1] == 8          # page-table epoch = pages
    assert d.exact_page_table_updates == 1
    assert d.tail_logical_begin == 6
    d.plan(8 * PAGE - 1)
    assert d.exact_page_table_updates == 1
    assert d.exact_table.last_len.tolist() == [15, 15]
    assert d.kernel_replans == 1                     # same structure: no re-plan
    assert len(d.decode.calls) == 1


def test_decoder_plan_fixed_suffix_uses_exact_once_tables():
    """reference tests/test_page_gauge_transformer.py:377-427 (tail 2, prefix
    1, static suffix 2, initial context 8 pages; capacity 12 here so that the
    tail can move past the suffix)."""
    d = _plan_only_decoder(batch=1, max_pages=12, tail_pages=2, sink_pages=1, suffix_pages=2,
                           initial=8)
    d.plan(8 * PAGE)
    old_indptr, old_indices, old_last, exact_indptr, exact_indices, exact_last = d.decode.calls[-1]
    assert old_indices == [1, 2, 3, 4, 5]
    assert exact_indices == [0, 1, 2]
    assert d.old_pages * PAGE == 5 * PAGE and d.exact_pages == 3
    d.plan(8 * PAGE + 1)
    old_indptr, old_indices, old_last, exact_indptr, exact_indices, exact_last = d.decode.calls[-1]
    assert old_indices == [1, 2, 3, 4, 5]
    assert exact_indices == [0, 1, 2, 3]
    assert len(set(exact_indices)) == 4
    assert d.old_pages + d.exact_pages == 9
    assert exact_last == [1]
    # the tail moves past the suffix; the suffix (pages 6, 7: slots 1, 2) stays
    d.plan(10 * PAGE)
    old_indices, exact_indices = d.decode.calls[-1][1], d.decode.calls[-1][4]
    assert old_indices == [1, 2, 3, 4, 5]
    assert exact_indices == [0, 1, 2, 3 + 8 % 2, 3 + 9 % 2]
    # one page later page 8 leaves the ring for the INT8 table
    d.plan(10 * PAGE + 1)
    old_indices, exact_indices = d.decode.calls[-1][1], d.decode.calls[-1][4]
    assert old_indices == [1, 2, 3, 4, 5, 8]
    assert exact_indices == [0, 1, 2, 3 + 9 % 2, 3 + 10 % 2]
    assert d.old_pages + d.exact_pages == 11
    assert d.old_page_table_updates == 2


def test_decoder_plan_replans_once_per_page_window():
    # 16 decode steps inside one page reuse one plan; the 17th crosses a page
    d = _plan_only_decoder(batch=1, max_pages=80, tail_pages=16, sink_pages=0)
    start = 64 * PAGE
    for position in range(start, start + PAGE):
        d.plan(position + 1)
    assert d.kernel_replans == 1
    assert d.old_pages == 65 - 16 and d.exact_pages == 16
    signature = d.plan_signature()
    d.plan(start + PAGE + 1)
    assert d.kernel_replans == 2 and d.plan_signature() != signature
    old_indptr, old_indices, _, _, exact_indices, exact_last = d.decode.calls[-1]
    assert old_indices == list(range(50))            # request-major identity pages
    assert exact_indices == [(p % 16) for p in range(50, 66)]   # ring slots, chronological
    assert exact_last == [1]


def test_plan_rejects_contexts_outside_the_cache():
    d = _plan_only_decoder(batch=1, max_pages=20, tail_pages=16, sink_pages=0)
    with pytest.raises(ValueError, match="outside the allocated cache capacity"):
        d.plan(21 * PAGE)
    with pytest.raises(ValueError, match="at least one quantized old page"):
        d.plan(16 * PAGE)


def test_rope_tables_match_transformers_rotary_embedding():
    from transformers import MistralConfig
    from transformers.models.mistral.modeling_mistral import MistralRotaryEmbedding

    cfg = MistralConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                        rope_theta=1.0e6, max_position_embeddings=4096)
    emb = MistralRotaryEmbedding(cfg)
    positions = torch.arange(3000)[None]
    cos, sin = emb(torch.zeros(1, 1, 4096), positions)
    got_cos, got_sin = dec.rope_tables(3000, 1.0e6)
    assert torch.equal(got_cos, cos[0].to(torch.float16))
    assert torch.equal(got_sin, sin[0].to(torch.float16))
    # closed form at one point: angle = p * theta^(-2i/128)
    p, i = 2999, 5
    assert abs(float(got_cos[p, i]) - math.cos(p * 1.0e6 ** (-2 * i / 128))) < 1e-3


def test_rms_norm_matches_transformers():
    from transformers.models.mistral.modeling_mistral import MistralRMSNorm

    norm = MistralRMSNorm(64, eps=1e-5).to(torch.float16)
    with torch.no_grad():
        norm.weight.copy_(torch.linspace(0.5, 1.5, 64))
    x = (torch.randn(3, 64, generator=torch.Generator().manual_seed(1)) * 3).to(torch.float16)
    assert torch.equal(dec.rms_norm(x, norm.weight.detach(), 1e-5), norm(x).detach())


def test_rope_is_the_append_kernel_formula():
    # x*c + rotate_half(x)*s with every product and the sum rounded to fp16
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(5, 2, 128, generator=gen).to(torch.float16)
    cos, sin = dec.rope_tables(5, 1.0e6)
    got = dec.rope(x, cos, sin)
    from oracle import pg_oracle as oracle
    for t in range(5):
        want = oracle.rope_rotate(x[t].numpy(), cos[t].numpy(), sin[t].numpy())
        assert (got[t].numpy().view("u2") == want.view("u2")).all()


def _tiny_config():
    return dec.DecoderConfig(layers=2, hidden=512, q_heads=4, kv_heads=1, intermediate=96,
                             vocab=80, rope_theta=1.0e4)


def test_prefill_matches_transformers_mistral():
    """Our prefill (fused projections, grouped attention, RoPE) equals
    ``MistralForCausalLM`` loaded with the same weights, in float32."""
    from transformers import MistralConfig, MistralForCausalLM

    cfg = _tiny_config()
    weights = dec.DecoderWeights(cfg, seed=7, device="cpu")
    hf = MistralForCausalLM(MistralConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
        num_hidden_layers=cfg.layers, num_attention_heads=cfg.q_heads,
        num_key_value_heads=cfg.kv_heads, rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_eps,
        max_position_embeddings=256, tie_word_embeddings=False, attn_implementation="eager"))
    qw, kw = cfg.q_heads * 128, cfg.kv_heads * 128
    with torch.no_grad():
        hf.model.embed_tokens.weight.copy_(weights.embed.float())
        for layer, w in zip(hf.model.layers, weights.layers):
            qkv = w["qkv"].float()
            layer.self_attn.q_proj.weight.copy_(qkv[:qw])
            layer.self_attn.k_proj.weight.copy_(qkv[qw:qw + kw])
            layer.self_attn.v_proj.weight.copy_(qkv[qw + kw:])
            layer.self_attn.o_proj.weight.copy_(w["o"].float())
            gate_up = w["gate_up"].float()
            layer.mlp.gate_proj.weight.copy_(gate_up[:cfg.intermediate])
            layer.mlp.up_proj.weight.copy_(gate_up[cfg.intermediate:])
            layer.mlp.down_proj.weight.copy_(w["down"].float())
        hf.lm_head.weight.copy_(weights.lm_head.float())
    hf.eval()
    tokens = torch.randint(0, cfg.vocab, (48,), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        want = hf(tokens[None]).logits[0, -1].float()
    # run our prefill in float32 (same code, weights cast)
    w32 = dec.DecoderWeights.__new__(dec.DecoderWeights)
    w32.config = cfg
    w32.embed = weights.embed.float()
    w32.layers = [{k: v.float() for k, v in w.items()} for w in weights.layers]
    w32.norm, w32.lm_head = weights.norm.float(), weights.lm_head.float()
    cos, sin = dec.rope_tables(48, cfg.rope_theta)
    captured = {}

    def on_layer(layer, key, value):
        captured[layer] = (key.clone(), value.clone())

    got = dec.prefill(w32, tokens, cos.float(), sin.float(), on_layer)[0]
    assert (got - want).abs().max() < 2e-3 * max(1.0, float(want.abs().max()))
    assert captured[0][0].shape == (48, cfg.kv_heads, 128)


def test_causal_attention_matches_naive_softmax():
    gen = torch.Generator().manual_seed(11)
    q = torch.randn(37, 8, 128, generator=gen)
    k = torch.randn(37, 2, 128, generator=gen)
    v = torch.randn(37, 2, 128, generator=gen)
    got = dec._causal_attention(q, k, v, chunk=16).float()
    for t in (0, 15, 16, 36):
        for h in (0, 3, 4, 7):
            g = h // 4
            s = (k[:t + 1, g] @ q[t, h]) / math.sqrt(128)
            p = torch.softmax(s.double(), 0)
            want = (p[:, None] * v[:t + 1, g].double()).sum(0)
            assert (got[t, h].double() - want).abs().max() < 1e-2


def test_decoder_config_rejects_unsupported_head_layouts():
    with pytest.raises(ValueError, match="head_dim 128 and GQA group 4"):
        dec.DecoderConfig(hidden=4096, q_heads=32, kv_heads=4)
    with pytest.raises(ValueError, match="head_dim 128"):
        dec.DecoderConfig(hidden=4000)


class _FakeUnified:
    def __init__(self):
        self.calls = []

    def plan(self, indptr, indices, last, *args, **kwargs):
        self.calls.append((indptr.tolist(), indices.tolist(), last.tolist()))


def test_heterogeneous_decoder_plan_writes_one_unified_table():
    # reference :2085-2110 and tests/test_page_gauge_transformer.py:199-216
    d = _plan_only_decoder(batch=2, max_pages=8, tail_pages=2, sink_pages=0)
    d.tail_attention = "heterogeneous"
    d.heterogeneous_pages = torch.empty_like(d.all_pages)
    d.old_kv_len = torch.zeros(2, dtype=torch.int32)
    d.heterogeneous_layout = None
    d.heterogeneous_page_table_updates = 0
    d.table = dec.SegmentTable(2, 8, "cpu")
    d.decode = _FakeUnified()
    d.plan(8 * PAGE)
    indptr, indices, last = d.decode.calls[-1]
    assert indptr == [0, 8, 16]
    assert indices == [0, 1, 2, 3, 4, 5, 0, 1, 8, 9, 10, 11, 12, 13, 2, 3]
    assert last == [16, 16] and d.old_kv_len.tolist() == [96, 96]
    d.plan(8 * PAGE - 3)                     # same layout: no new table, no new plan
    assert d.heterogeneous_page_table_updates == 1 and d.kernel_replans == 1
    assert d.table.last_len.tolist() == [13, 13]
    d.plan(7 * PAGE)                         # one page less: new layout
    assert d.heterogeneous_page_table_updates == 2 and d.kernel_replans == 2
    assert d.decode.calls[-1][1] == [0, 1, 2, 3, 4, 1, 0, 8, 9, 10, 11, 12, 3, 2]
    assert d.old_kv_len.tolist() == [80, 80]
