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

import math

import pytest
import torch
import torch.nn.functional as F

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


def _dense_reference_class(dec):
    class DenseReference(dec.PageGaugeDecoder):
        """Attention = float32 softmax over K = c_K + s*Z (old) / c_K + ring
        (tail), V likewise, from the same cache the K2 kernel updates.  The
        PageGauge kernel runs on the same inputs first; ``kernel_error``
        records max |kernel - dense| - half an FP16 ulp of the dense value
        (the kernel's output rounding)."""

        kernel_error = 0.0

        def attention(self, layer):
            kernel = super().attention(layer).float().clone()
            dense = self._dense(layer)
            excess = (kernel - dense).abs() - dense.abs() * 2.0 ** -11
            self.kernel_error = max(self.kernel_error, float(excess.max()))
            self.attention_output[layer].copy_(dense.to(torch.float16))
            return self.attention_output[layer]

        def _dense(self, layer):
            c = self.cache
            b = 0
            old = self.old_table.active_indices().long()
            tail = self.exact_table.active_indices().long()
            last = int(self.exact_table.host_last_len[b])
            kc = c.key_center[layer, b].float()
            vc = c.value_center[layer, b].float()
            k_old = c.key_codes[layer][old].float() * c.key_scales[layer][old].float()[:, None, :, None]
            v_old = c.value_codes[layer][old].float() * c.value_scales[layer][old].float()[:, None, :, None]
            k_tail = c.exact_key[layer][tail].float()
            v_tail = c.exact_value[layer][tail].float()
            n_tail = (tail.numel() - 1) * 16 + last
            keys = torch.cat((k_old.reshape(-1, 8, 128), k_tail.reshape(-1, 8, 128)[:n_tail])) + kc
            values = torch.cat((v_old.reshape(-1, 8, 128), v_tail.reshape(-1, 8, 128)[:n_tail])) + vc
            q = self.rotated_query[b].float().view(8, 4, 128)
            scores = torch.matmul(q, keys.permute(1, 2, 0).contiguous()) / math.sqrt(128)
            probs = torch.softmax(scores, dim=-1)
            return torch.matmul(probs, values.permute(1, 0, 2).contiguous()).reshape(1, 32, 128)

    return DenseReference


def test_page_gauge_logits_match_dense_reference(setup):
    """Per layer and step, the K1 output on the reference decoder's own
    inputs is within 2e-3 (+ half an FP16 ulp of output rounding) of the
    dense float32 attention; the logits of the PageGauge decoder and of the
    dense-attention decoder (whose states drift apart by FP16 roundings over
    20 steps of 2 layers) stay within 8 * 2e-3."""
    dec, weights, first, decoders, tokens = setup
    pg = _fresh(dec, decoders["page_gauge"])
    ref = _fresh(dec, decoders["page_gauge"], _dense_reference_class(dec))
    worst_logit = 0.0
    for i in range(STEPS):
        position = PROMPT + i
        got = pg.step(tokens[i:i + 1], position).clone()
        want = ref.step(tokens[i:i + 1], position)
        worst_logit = max(worst_logit, float((got - want).abs().max()))
    print(f"attention: max excess over half-ulp |kernel - dense| = {ref.kernel_error:.3g}; "
          f"max |logits - dense decoder| = {worst_logit:.3g}")
    assert ref.kernel_error <= 2e-3
    assert worst_logit <= 2e-3 * 8


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
