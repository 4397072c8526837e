"""The decoder over the PageGauge kernels on the GPU (a reduced Mistral: the
full 32/8-head, head-dim-128 layout, 2 layers, small MLP and vocabulary).

* PageGauge logits against the same decoder whose attention is the dense
  float32 softmax over the reconstructed cache (the reference's own path,
  diagnostics/benchmark_heterogeneous_fa2_correctness.py:291-299);
* PageGauge against the FP16-cache decoder: the reference's acceptance gate
  (logit cosine >= 0.995 and top-1 agreement,
  scripts/benchmark_page_gauge_transformer.py:3865-3903);
* graph replay bitwise equal to eager steps, a page transition that misses
  the graph bank and runs eagerly (:3706-3860), and greedy generation."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import dense_reference_class

pytestmark = pytest.mark.gpu

PROMPT = 512           # 32 pages: 16 INT8 + 16 FP16 tail
STEPS = 20             # crosses one page boundary (positions 512..531)


@pytest.fixture(scope="module")
def setup(cuda):
    from pagegauge_amd import decoder as dec

    cfg = dec.DecoderConfig(layers=2, intermediate=512, vocab=1024)
    weights = dec.DecoderWeights(cfg, seed=20260850, device=cuda)
    gen = torch.Generator().manual_seed(20260850)
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=gen)
    first, logits, decoders = dec.build_decoders(weights, prompt, STEPS + 1)
    tokens = torch.randint(0, cfg.vocab, (STEPS,), generator=gen).to(cuda)
    torch.cuda.synchronize()
    return dec, weights, first, decoders, tokens


def _fresh(dec, base, backend=None):
    """A decoder over a private copy of ``base``'s cache."""
    cls = type(base) if backend is None else backend
    d = cls(base.weights, base.cache.clone(), base.backend, base.max_pages * 16, base.rope_cos,
            base.rope_sin, base.exact_tail_pages * 16, base.split_pages, base.batch_size,
            base.exact_sink_pages)
    return d


FLOOR_BOUND = 1e-2     # the 2-layer decoder's FP16 rounding floor measured 6.4e-3


def test_page_gauge_logits_within_the_fp16_floor_of_dense_reference(setup):
    """At every one of 20 positions, from one cache state, one PageGauge
    step against the same step whose attention is the dense float32 softmax
    over the reconstructed cache: the K1 output on the same inputs is within
    2e-3 (+ half an FP16 ulp of output rounding) of the dense attention, and
    the logits are within max(2e-3, floor), where the floor is what the same
    step's logits move between an O projection fed the float32 dense attention
    and one fed its FP16 rounding (the decoder's own rounding floor).  The
    floor must stay below a bound pinned from measured runs, so that the gate
    cannot widen unnoticed."""
    dec, weights, first, decoders, tokens = setup
    walker = _fresh(dec, decoders["page_gauge"])
    dense32 = dense_reference_class(dec)
    rounded = dense_reference_class(dec, torch.float64, attention_output="float16")
    unrounded = dense_reference_class(dec, torch.float64, attention_output="float32")
    worst, floor, kernel = 0.0, 0.0, 0.0
    for i in range(STEPS):
        position = PROMPT + i
        pg = _fresh(dec, walker)
        ref = _fresh(dec, walker, dense32)
        f16 = _fresh(dec, walker, rounded)
        f32 = _fresh(dec, walker, unrounded)
        got = pg.step(tokens[i:i + 1], position).clone()
        want = ref.step(tokens[i:i + 1], position).clone()
        a = f16.step(tokens[i:i + 1], position).clone()
        b = f32.step(tokens[i:i + 1], position)
        worst = max(worst, float((got - want).abs().max()))
        floor = max(floor, float((a - b).abs().max()))
        kernel = max(kernel, ref.kernel_error)
        walker.step(tokens[i:i + 1], position)
    print(f"attention: max excess over half-ulp |kernel - dense| = {kernel:.3g}; "
          f"max |logits - dense decoder| = {worst:.3g}; floor = {floor:.3g}")
    assert kernel <= 2e-3
    assert floor <= FLOOR_BOUND
    assert worst <= max(2e-3, floor)


def test_page_gauge_agrees_with_fp16_cache_decoder(setup):
    dec, weights, first, decoders, tokens = setup
    pg = _fresh(dec, decoders["page_gauge"])
    fp = _fresh(dec, decoders["fp16"])
    cosines, top1 = [], []
    for i in range(STEPS):
        a = pg.step(tokens[i:i + 1], PROMPT + i).clone()
        b = fp.step(tokens[i:i + 1], PROMPT + i)
        cosines.append(float(F.cosine_similarity(a, b, dim=-1).min()))
        top1.append(bool((a.argmax(-1) == b.argmax(-1)).all()))
    print(f"min cosine {min(cosines):.6f}, top-1 agreement {sum(top1)}/{len(top1)}")
    assert min(cosines) >= 0.995
    assert sum(top1) >= 0.8 * len(top1)


@pytest.mark.parametrize("backend", ["page_gauge", "fp16"])
def test_graph_replay_is_bitwise_eager_and_transitions_run_eagerly(setup, backend):
    dec, weights, first, decoders, tokens = setup
    eager = _fresh(dec, decoders[backend])
    graphed = _fresh(dec, decoders[backend])
    window = 16
    want = [eager.step(tokens[i:i + 1], PROMPT + i).clone() for i in range(window + 1)]
    graphed.capture(PROMPT)
    replays = []
    for i in range(window):
        replays.append(graphed.step(tokens[i:i + 1], PROMPT + i).clone())
        torch.cuda.synchronize()                     # eager host work between replays
    counts = graphed.counts()
    assert counts["graph_replays"] == window and counts["eager_steps"] == 0
    for i in range(window):
        assert torch.equal(replays[i], want[i]), f"step {i}"
    # the next token opens a new page: new plan signature, no banked graph
    transition = graphed.step(tokens[window:window + 1], PROMPT + window)
    assert graphed.counts()["graph_bank_misses"] == 1
    assert torch.equal(transition, want[window])


def test_heterogeneous_decoder_matches_segmented_and_replays(setup):
    """tail_attention='heterogeneous' (one unified table, old_kv_len on the
    device) gives the segmented decoder's logits up to accumulation order,
    and its whole-step graph replays bitwise."""
    dec, weights, first, decoders, tokens = setup
    base = decoders["page_gauge"]

    def make(tail):
        return dec.PageGaugeDecoder(weights, base.cache.clone(), "page_gauge", base.max_pages * 16,
                                    base.rope_cos, base.rope_sin, tail_attention=tail)

    seg, het, het_graph = make("segmented"), make("heterogeneous"), make("heterogeneous")
    het_graph.capture(PROMPT)
    for i in range(STEPS):
        a = seg.step(tokens[i:i + 1], PROMPT + i).clone()
        b = het.step(tokens[i:i + 1], PROMPT + i).clone()
        c = het_graph.step(tokens[i:i + 1], PROMPT + i)
        assert float((a - b).abs().max()) <= 2e-2, i
        assert float(torch.nn.functional.cosine_similarity(a, b, dim=-1).min()) > 0.99999
        if i < 16:
            assert torch.equal(b, c), i
    assert het.counts()["table"]["plan_rebuilds"] == 2     # one page window, then the next


def test_greedy_generation_graph_equals_eager(setup):
    dec, weights, first, decoders, tokens = setup
    a = _fresh(dec, decoders["page_gauge"])
    b = _fresh(dec, decoders["page_gauge"])
    toks_graph, logits_graph = a.generate(first, PROMPT, STEPS, use_graphs=True)
    toks_eager, logits_eager = b.generate(first, PROMPT, STEPS, use_graphs=False)
    assert torch.equal(toks_graph, toks_eager)
    for x, y in zip(logits_graph, logits_eager):
        assert torch.equal(x, y)
    assert a.counts()["graph_replays"] == STEPS
    assert len(a.graph_bank) == 2                     # one per page window


def test_decoder_requires_the_hip_library(setup, monkeypatch):
    from pagegauge_amd import _capi

    from pagegauge_amd import runtime

    dec, weights, first, decoders, tokens = setup
    monkeypatch.setattr(_capi, "_library", None)
    monkeypatch.setattr(_capi, "LIBRARY_PATH", _capi.LIBRARY_PATH.with_name("absent.so"))
    monkeypatch.setattr(runtime, "_EXTENSION", None)
    with pytest.raises(_capi.LibraryMissingError):
        _fresh(dec, decoders["page_gauge"])
    with pytest.raises(_capi.LibraryMissingError):
        decoders["page_gauge"].step(tokens[:1], PROMPT)     # its first plan needs the library


def _cache_tensors(cache):
    return {k: v for k, v in vars(cache).items() if isinstance(v, torch.Tensor)}


@pytest.mark.parametrize("backend,tail,sink", [("page_gauge", "segmented", 0),
                                               ("page_gauge", "heterogeneous", 0),
                                               ("fp16", "segmented", 0),
                                               ("page_gauge", "segmented", 2)])
def test_fused_cache_update_is_bitwise_the_separate_update(setup, backend, tail, sink):
    """The QKV projection carrying RoPE + append (pg_decoder_qkv_rope_append)
    and the decode's finalize of a completed page (pg_decode_run_finalize)
    leave the caches and logits bit-identical to the projection followed by
    the K2 launch, across a page completion (position 527)."""
    dec, weights, first, decoders, tokens = setup
    if sink:
        gen = torch.Generator().manual_seed(20260850)
        prompt = torch.randint(0, weights.config.vocab, (PROMPT,), generator=gen)
        _, _, built = dec.build_decoders(weights, prompt, STEPS + 1, backends=("page_gauge",),
                                         exact_sink_pages=sink)
        base = built["page_gauge"]
    else:
        base = decoders[backend]

    def make(fused_append):
        return dec.PageGaugeDecoder(weights, base.cache.clone(), backend, base.max_pages * 16,
                                    base.rope_cos, base.rope_sin, base.exact_tail_pages * 16,
                                    exact_sink_pages=base.exact_sink_pages, tail_attention=tail,
                                    fused_append=fused_append)

    fused, separate = make(True), make(False)
    assert fused.fused_append and not separate.fused_append
    for i in range(STEPS):
        a = fused.step(tokens[i:i + 1], PROMPT + i).clone()
        b = separate.step(tokens[i:i + 1], PROMPT + i)
        assert torch.equal(a, b), f"logits differ at step {i}"
    for name, value in _cache_tensors(fused.cache).items():
        assert torch.equal(value, _cache_tensors(separate.cache)[name]), name
    if backend == "page_gauge":
        # the page completed at position 527 (logical page 32) was finalized
        assert fused.cache.key_scales[:, 32].abs().min() > 0


def test_batched_decoder_steps_requests_in_lockstep(setup):
    """build_decoders over a [2, T] prompt (one prefill per request, each into
    its own cache slot): two copies of the same prompt give bitwise the same
    logits for both requests at every step, and they match the one-request
    decoder (the split plans differ, so within the attention tolerance)."""
    dec, weights, first, decoders, tokens = setup
    cfg = weights.config
    gen = torch.Generator().manual_seed(20260850)
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=gen)
    print("batched decoder B=2", flush=True)
    first2, logits2, built = dec.build_decoders(weights, torch.stack((prompt, prompt)), STEPS + 1,
                                                backends=("page_gauge",))
    batched = built["page_gauge"]
    single = _fresh(dec, decoders["page_gauge"])
    assert batched.batch_size == 2 and torch.equal(first2, first.repeat(2))
    for i in range(STEPS):
        pair = batched.step(tokens[i].repeat(2), PROMPT + i).clone()
        one = single.step(tokens[i:i + 1], PROMPT + i).clone()
        assert torch.equal(pair[0], pair[1]), i
        assert float((pair[:1] - one).abs().max()) <= 1.6e-2, i
