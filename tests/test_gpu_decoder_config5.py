"""Config 5 at its own shape: the full Mistral-7B-architecture decoder.

Random-init fp16 weights (seed 20260850; 32 layers, hidden 4096, 32/8 heads,
MLP 14336, vocab 32768, RoPE theta 1e6), a 16384-token prompt of uniform
random ids prefilled into the PageGauge cache (INT8 pages + 256-token FP16
ring) and into an FP16 cache, then decode steps at positions 16384....

* Logits (within 2e-3 of the reference's own path).
  From one cache state, one PageGauge step is compared with the same step
  whose attention is the dense float32 softmax over the reconstructed cache
  (the reference's explicit-reconstruction path), at positions 16384-16387,
  at 16399 (its token completes page 1024, which K1's FP16 pass quantizes in
  the same step) and at 16400 (the ring slot of page 1009 is reused: the
  INT8 segment grows by that page, quantized during the prefill).  The
  resolution of that comparison is the FP16 rounding floor of the decoder
  itself: the logits of the same step move by that much between an O
  projection fed the float32 dense attention and one fed its FP16 rounding
  (the reference's kernels also return FP16 attention).  The gate is
  max(2e-3, the largest floor of the checked steps), and that floor must stay
  below a bound pinned from measured runs (3.32e-2 measured over these six
  steps; bound 4e-2), so a change in the reference helpers cannot widen the
  gate unnoticed.  The
  north star's literal 2e-3 is met by the attention (``kernel_error``), not
  by the 32-layer logits, which cannot resolve it.
* The reference's acceptance gate against the FP16-cache decoder (logit
  cosine >= 0.995, top-1 agreement >= 80 %,
  scripts/benchmark_page_gauge_transformer.py:3865-3903).
* Whole-step graph replay bitwise equal to eager steps.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import dense_reference_class

pytestmark = pytest.mark.gpu

PROMPT = 16384
STEPS = 4              # graph steps
AGREE_STEPS = 16       # teacher-forced steps of the cosine / top-1 gate, as in bench.py
# logits positions: the first steps, the page-closing step and the one after it
LOGIT_POSITIONS = (PROMPT, PROMPT + 1, PROMPT + 2, PROMPT + 3, PROMPT + 15, PROMPT + 16)
FLOOR_BOUND = 4e-2     # the decoder's FP16 rounding floor measured 3.32e-2 at this shape


@pytest.fixture(scope="module")
def full(cuda):
    from pagegauge_amd import decoder as dec

    cfg = dec.DecoderConfig()
    weights = dec.DecoderWeights(cfg, seed=20260850, device=cuda)
    gen = torch.Generator().manual_seed(20260850)
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=gen)
    tokens = torch.randint(0, cfg.vocab, (AGREE_STEPS + 1,), generator=gen).to(cuda)
    print("config5: prefill of 16384 tokens, 32 layers", flush=True)
    first, _, decoders = dec.build_decoders(weights, prompt, AGREE_STEPS + 1)
    torch.cuda.synchronize()
    yield dec, weights, decoders, tokens
    del decoders, weights
    torch.cuda.empty_cache()


def _make(dec, base, cls=None, cache=None):
    cls = type(base) if cls is None else cls
    return cls(base.weights, (base.cache if cache is None else cache).clone(), base.backend,
               base.max_pages * 16, base.rope_cos, base.rope_sin, base.exact_tail_pages * 16,
               base.split_pages, base.batch_size, base.exact_sink_pages)


def test_config5_logits_within_the_fp16_floor_of_dense_reference(full):
    dec, weights, decoders, tokens = full
    walker = _make(dec, decoders["page_gauge"])     # advances the shared cache state
    dense32 = dense_reference_class(dec)
    rounded = dense_reference_class(dec, torch.float64, attention_output="float16")
    unrounded = dense_reference_class(dec, torch.float64, attention_output="float32")
    rows = []
    for position in range(PROMPT, LOGIT_POSITIONS[-1] + 1):
        i = position - PROMPT
        if position in LOGIT_POSITIONS:
            state = walker.cache
            pg = _make(dec, walker, cache=state)
            ref = _make(dec, walker, dense32, cache=state)
            f16 = _make(dec, walker, rounded, cache=state)
            f32 = _make(dec, walker, unrounded, cache=state)
            got = pg.step(tokens[i:i + 1], position).clone()
            want = ref.step(tokens[i:i + 1], position).clone()
            a = f16.step(tokens[i:i + 1], position).clone()
            b = f32.step(tokens[i:i + 1], position).clone()
            row = (position, float((got - want).abs().max()), float((a - b).abs().max()),
                   ref.kernel_error)
            rows.append(row)
            del pg, ref, f16, f32
            print(f"config5 position {position}{' (page closes)' if position % 16 == 15 else ''}: "
                  f"max|pg - dense| {row[1]:.3g}, FP16 rounding floor {row[2]:.3g}, "
                  f"attention excess {row[3]:.3g}", flush=True)
        walker.step(tokens[i:i + 1], position)
    # one gate for every position: the floor is one sample per step of the
    # same FP16 rounding effect the distance measures, so a step is held to
    # the largest floor of the checked steps (as over 16384-16387 before)
    floor = max(row[2] for row in rows)
    print(f"config5 gate max(2e-3, floor) = {max(2e-3, floor):.3g}", flush=True)
    assert floor <= FLOOR_BOUND
    for position, distance, _, kernel in rows:
        assert kernel <= 2e-3, position
        assert distance <= max(2e-3, floor), position


def test_config5_cosine_and_top1_against_fp16_cache(full):
    dec, weights, decoders, tokens = full
    pg = _make(dec, decoders["page_gauge"])
    fp = _make(dec, decoders["fp16"])
    cosines, top1 = [], []
    for i in range(AGREE_STEPS):
        a = pg.step(tokens[i:i + 1], PROMPT + i).clone()
        b = fp.step(tokens[i:i + 1], PROMPT + i)
        cosines.append(float(F.cosine_similarity(a, b, dim=-1).min()))
        top1.append(bool((a.argmax(-1) == b.argmax(-1)).all()))
    print(f"config5 min cosine {min(cosines):.6f}, top-1 {sum(top1)}/{len(top1)}", flush=True)
    assert min(cosines) >= 0.995
    assert sum(top1) >= 0.8 * len(top1)


def test_config5_graph_replay_is_bitwise_eager(full):
    dec, weights, decoders, tokens = full
    eager = _make(dec, decoders["page_gauge"])
    graphed = _make(dec, decoders["page_gauge"])
    want = [eager.step(tokens[i:i + 1], PROMPT + i).clone() for i in range(STEPS)]
    graphed.capture(PROMPT)
    for i in range(STEPS):
        got = graphed.step(tokens[i:i + 1], PROMPT + i).clone()
        torch.cuda.synchronize()                     # eager host work between replays
        assert torch.equal(got, want[i]), f"step {i}"
    assert graphed.counts()["graph_replays"] == STEPS
