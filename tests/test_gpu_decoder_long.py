"""A long decode with the reduced decoder (the full 32/8-head, head-dim-128
layout, 2 layers): 320 steps from a 512-token prompt cross 20 page
boundaries, so the 16-page FP16 ring wraps (from position 768 on) and every
page a step completes is finalized into INT8 codes by K1's FP16 pass while
the following steps read it as history.  Checked over the whole run:

* the PageGauge decoder against the FP16-cache decoder, teacher-forced: the
  reference's acceptance gate (logit cosine >= 0.995, top-1 agreement >= 80 %,
  scripts/benchmark_page_gauge_transformer.py:3865-3903) at every step --
  the FP16 cache does not share the INT8 tables, so a table or ring error
  would show here;
* K1 against the dense float32 softmax over the reconstructed cache on the
  same inputs, at every step (within 2e-3 beyond half an FP16 ulp);
* greedy generation with one graph per page window, bitwise equal to eager
  steps."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import dense_reference_class

pytestmark = pytest.mark.gpu

PROMPT = 512           # 32 pages: 16 INT8 + the 16-page FP16 ring
STEPS = 320            # positions 512..831: 20 page boundaries, the ring wraps


@pytest.fixture(scope="module")
def setup(cuda):
    from pagegauge_amd import decoder as dec

    cfg = dec.DecoderConfig(layers=2, intermediate=512, vocab=1024)
    weights = dec.DecoderWeights(cfg, seed=20260851, device=cuda)
    gen = torch.Generator().manual_seed(20260851)
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=gen)
    first, _, decoders = dec.build_decoders(weights, prompt, STEPS + 1)
    tokens = torch.randint(0, cfg.vocab, (STEPS,), generator=gen).to(cuda)
    torch.cuda.synchronize()
    return dec, first, decoders, tokens


def _fresh(base, cls=None):
    cls = type(base) if cls is None else cls
    return cls(base.weights, base.cache.clone(), base.backend, base.max_pages * 16, base.rope_cos,
               base.rope_sin, base.exact_tail_pages * 16, base.split_pages, base.batch_size,
               base.exact_sink_pages)


def test_long_teacher_forced_decode_tracks_the_fp16_cache_decoder(setup):
    dec, first, decoders, tokens = setup
    pg = _fresh(decoders["page_gauge"])
    fp = _fresh(decoders["fp16"])
    cosines, top1 = [], []
    for i in range(STEPS):
        a = pg.step(tokens[i:i + 1], PROMPT + i).clone()
        b = fp.step(tokens[i:i + 1], PROMPT + i)
        cosines.append(float(F.cosine_similarity(a, b, dim=-1).min()))
        top1.append(bool((a.argmax(-1) == b.argmax(-1)).all()))
    worst = min(range(STEPS), key=lambda i: cosines[i])
    print(f"min cosine {cosines[worst]:.6f} at position {PROMPT + worst}, "
          f"top-1 agreement {sum(top1)}/{STEPS}", flush=True)
    assert cosines[worst] >= 0.995
    assert sum(top1) >= 0.8 * STEPS
    # the plan followed every page window (one rebuild per new page)
    assert pg.counts()["old_table"]["plan_rebuilds"] >= 20


def test_long_decode_kernel_matches_dense_attention_at_every_step(setup):
    dec, first, decoders, tokens = setup
    ref = _fresh(decoders["page_gauge"], dense_reference_class(dec))
    worst = 0.0
    for i in range(STEPS):
        ref.step(tokens[i:i + 1], PROMPT + i)
        worst = max(worst, ref.kernel_error)
    print(f"max excess over half-ulp |kernel - dense| over {STEPS} steps: {worst:.3g}", flush=True)
    assert worst <= 2e-3


def test_long_greedy_generation_graph_equals_eager(setup):
    dec, first, decoders, tokens = setup
    a = _fresh(decoders["page_gauge"])
    b = _fresh(decoders["page_gauge"])
    toks_graph, logits_graph = a.generate(first, PROMPT, STEPS, use_graphs=True)
    toks_eager, logits_eager = b.generate(first, PROMPT, STEPS, use_graphs=False)
    assert torch.equal(toks_graph, toks_eager)
    for x, y in zip(logits_graph, logits_eager):
        assert torch.equal(x, y)
    assert a.counts()["graph_replays"] == STEPS
    assert len(a.graph_bank) >= 20                     # one per page window
