"""The decoder with the reference's full exact-page policy: an exact prefix
(sink, S), a static exact suffix of the prefill (A), and the FP16 tail ring
(T) (scripts/benchmark_page_gauge_transformer.py:334-373, :460-749,
:1603-1642, :2034-2155).  A reduced Mistral (the full 32/8-head layout, 2
layers) with S = 1, A = 4 pages before the 32-page prompt's end and an
8-page ring, decoded for 140 steps: the ring first overlaps the suffix, then
moves past it; prefill pages leave the ring for the INT8 table (page 24 at
the first step), the suffix pages never do, and the pages the decode itself
completes and finalizes leave the ring from position 640 on.

* At every step, K1's output against the dense float32 softmax over the
  context rebuilt from the page classes (every logical page once, from the
  INT8 pool or its exact slot; not from the decoder's tables): within 2e-3
  beyond half an FP16 ulp of the dense value.
* At positions across those transitions, the logits against the same step
  with dense attention, within max(2e-3, the decoder's FP16 rounding floor).
* The suffix slots hold the prefill's rows after 140 steps (no ring write
  lands on them), and graph replay equals eager steps bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from tests.helpers import dense_reference_class

pytestmark = pytest.mark.gpu

PROMPT = 512            # 32 pages
STEPS = 140             # positions 512..651
SINK, SUFFIX, TAIL = 1, 4, 128
LOGIT_POSITIONS = (512, 513, 527, 528, 575, 576, 639, 640, 651)
FLOOR_BOUND = 1e-2


@pytest.fixture(scope="module")
def setup(cuda):
    from pagegauge_amd import decoder as dec

    cfg = dec.DecoderConfig(layers=2, intermediate=512, vocab=1024)
    weights = dec.DecoderWeights(cfg, seed=20260850, device=cuda)
    gen = torch.Generator().manual_seed(20260851)
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=gen)
    tokens = torch.randint(0, cfg.vocab, (STEPS,), generator=gen).to(cuda)
    print(f"static suffix: S={SINK} A={SUFFIX} ring {TAIL // 16} pages, {STEPS} steps", flush=True)
    _, _, built = dec.build_decoders(weights, prompt, STEPS + 1, exact_tail=TAIL,
                                     backends=("page_gauge",), exact_sink_pages=SINK,
                                     exact_static_suffix_pages=SUFFIX)
    torch.cuda.synchronize()
    return dec, built["page_gauge"], tokens


def _copy(dec, base, cls=None, cache=None):
    cls = type(base) if cls is None else cls
    return cls(base.weights, (base.cache if cache is None else cache).clone(), base.backend,
               base.max_pages * 16, base.rope_cos, base.rope_sin, base.exact_tail_pages * 16,
               base.split_pages, base.batch_size, base.exact_sink_pages,
               exact_static_suffix_pages=base.exact_static_suffix_pages,
               initial_context_pages=base.initial_context_pages)


def test_suffix_layout(setup):
    dec, base, tokens = setup
    assert base.exact_fixed_pages == SINK + SUFFIX
    assert base.cache.exact_storage_pages_per_request == SINK + SUFFIX + TAIL // 16
    assert base.initial_context_pages == PROMPT // 16


def test_static_suffix_decode_against_dense_attention(setup):
    dec, base, tokens = setup
    walker = _copy(dec, base, dense_reference_class(dec, tables="logical"))
    suffix_slots = list(range(SINK, SINK + SUFFIX))
    suffix_rows = walker.cache.exact_key[:, suffix_slots].clone()
    dense32 = dense_reference_class(dec, tables="logical")
    rounded = dense_reference_class(dec, torch.float64, attention_output="float16", tables="logical")
    unrounded = dense_reference_class(dec, torch.float64, attention_output="float32",
                                      tables="logical")
    rows = []
    for i in range(STEPS):
        position = PROMPT + i
        if position in LOGIT_POSITIONS:
            state = walker.cache
            pg = _copy(dec, walker, dec.PageGaugeDecoder, cache=state)   # the product step
            ref = _copy(dec, walker, dense32, cache=state)
            f16 = _copy(dec, walker, rounded, cache=state)
            f32 = _copy(dec, walker, unrounded, cache=state)
            got = pg.step(tokens[i:i + 1], position).clone()
            want = ref.step(tokens[i:i + 1], position).clone()
            a = f16.step(tokens[i:i + 1], position).clone()
            b = f32.step(tokens[i:i + 1], position).clone()
            rows.append((position, float((got - want).abs().max()), float((a - b).abs().max())))
            print(f"position {position}: old {ref.old_pages} exact {ref.exact_pages} pages, "
                  f"max|pg - dense| {rows[-1][1]:.3g}, floor {rows[-1][2]:.3g}, "
                  f"attention excess {ref.kernel_error:.3g}", flush=True)
            assert ref.kernel_error <= 2e-3, position
            del pg, ref, f16, f32
        walker.step(tokens[i:i + 1], position)
        assert walker.kernel_error <= 2e-3, position          # K1 against dense, every step
    print(f"worst attention excess over {STEPS} steps: {walker.kernel_error:.3g}", flush=True)
    for position, distance, floor in rows:
        assert floor <= FLOOR_BOUND, position
        assert distance <= max(2e-3, floor), position
    # the suffix slots were never written by the ring
    assert torch.equal(walker.cache.exact_key[:, suffix_slots], suffix_rows)
    # the tail has moved past the suffix: pages 24..27 and the decode's first
    # completed pages are INT8 now, the suffix pages are not
    assert walker.old_pages + walker.exact_pages == walker.current_pages
    assert walker.exact_pages == SINK + SUFFIX + TAIL // 16


def test_static_suffix_graph_replay_is_bitwise_eager(setup):
    dec, base, tokens = setup
    eager = _copy(dec, base)
    graphed = _copy(dec, base)
    window = 20
    want = [eager.step(tokens[i:i + 1], PROMPT + i).clone() for i in range(window)]
    graphed.capture(PROMPT)
    for i in range(window):
        got = graphed.step(tokens[i:i + 1], PROMPT + i).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want[i]), f"step {i}"
