"""How often the reference's center formula and this build's exact center differ.

The reference computes a channel center as
``values.float().mean(dim=(0, 1)).half()``
(scripts/benchmark_flashinfer_page_affine_int8.py:262): a float32 reduction
in an unspecified order, then rounding to FP16.  This build defines the center
as the exact mean rounded once to float32 and once to FP16
(``oracle.exact_center``, the kernels' ``token_major_centers``), so that the
GPU result does not depend on a reduction order.  Every code of a page
follows from its center, so this test counts, on the bench's own data, the
center elements where the two definitions round to different FP16 values,
and checks that each such difference is one FP16 step.

Data: the K/V contexts of config 2 (B1/49K, seed 20260840, generated as the
bench line generates them, with the FP16 same-way copy) and config 3 (B8
ragged, the bench's three seeds), replayed from the same seeded generator on
the CPU; and, for config 5's per-layer shape (16,384 tokens x 8 KV heads x
128), four seeded N(0,1) layers standing in for the decoder's prefill K/V,
which a random-init model computes on the GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from pagegauge_amd import workloads as wl


def _contexts(lengths, seed, with_fp16_copy):
    """The per-request (keys, values) of ``workloads.build_decode_workload``:
    the same generator calls in the same order, host side only."""
    g = torch.Generator().manual_seed(seed)
    torch.randn(len(lengths), wl.HQ, wl.DIM, generator=g)                 # queries
    tail_pages = wl.TAIL_TOKENS // wl.PAGE
    total_old = sum(n // wl.PAGE - tail_pages for n in lengths)
    total_tail = tail_pages * len(lengths)
    torch.randperm(total_old, generator=g)
    torch.randperm(total_tail, generator=g)
    if with_fp16_copy:
        torch.randperm(total_old + total_tail, generator=g)
    for n in lengths:
        keys = wl._outlier_kv(g, n, 4, 8.0)
        values = wl._outlier_kv(g, n, 4, 8.0)
        yield keys, values


def _compare(tokens: torch.Tensor):
    """(elements, differing, max step) between the reference formula on the
    CPU and the exact center, for one [tokens, 8, 128] FP16 context."""
    pages = tokens.reshape(-1, wl.PAGE, *tokens.shape[1:])          # [pages, 16, 8, 128]
    ref = pages.float().mean(dim=(0, 1)).half().numpy()
    exact = oracle.exact_center(pages.numpy())
    a = ref.view(np.int16).astype(np.int32)
    b = exact.view(np.int16).astype(np.int32)
    # adjacent FP16 values of one sign differ by 1 in their bit patterns
    differ = a != b
    same_sign = np.sign(ref.astype(np.float32)) == np.sign(exact.astype(np.float32))
    steps = np.where(differ & same_sign, np.abs(a - b), np.where(differ, 99, 0))
    return int(ref.size), int(differ.sum()), int(steps.max())


def _tally(pairs):
    elements = differing = worst = 0
    for keys, values in pairs:
        for tokens in (keys, values):
            n, d, s = _compare(tokens)
            elements, differing, worst = elements + n, differing + d, max(worst, s)
    return elements, differing, worst


def test_exact_center_reduces_like_the_reference_mean_on_a_small_case():
    """The comparison helper itself: on 16 tokens whose float32 sum is exact,
    both definitions agree bit for bit."""
    t = torch.tensor([[[1.0, -2.0]], [[0.5, 0.25]], [[0.25, 0.125]], [[-0.75, 1.5]]],
                     dtype=torch.float16)
    t = t.expand(4, 8, 2).repeat(4, 1, 1).contiguous()              # 16 tokens
    n, d, s = _compare(t)
    assert (n, d, s) == (16, 0, 0)


@pytest.mark.parametrize("config,lengths_seeds", [
    ("config2_b1_49k", [([49152], 20260840)]),
    ("config3_b8_ragged", [(wl.ragged_lengths(s), s) for s in wl.VALIDATION_SEEDS[:3]]),
])
def test_reference_center_formula_against_exact_center(config, lengths_seeds, capsys):
    elements = differing = worst = 0
    for lengths, seed in lengths_seeds:
        n, d, s = _tally(_contexts(lengths, seed, with_fp16_copy=True))
        elements, differing, worst = elements + n, differing + d, max(worst, s)
    with capsys.disabled():
        print(f"\n{config}: {differing} of {elements} center elements differ "
              f"(largest difference {worst} FP16 step{'s' if worst != 1 else ''})")
    assert worst <= 1                      # never more than one FP16 step apart
    assert differing <= elements // 500    # rare: a half-way case of the FP16 rounding


def test_reference_center_formula_at_the_config5_layer_shape(capsys):
    g = torch.Generator().manual_seed(20260850)
    layers = ((torch.randn(16384, wl.HKV, wl.DIM, generator=g).half(),
               torch.randn(16384, wl.HKV, wl.DIM, generator=g).half()) for _ in range(4))
    elements, differing, worst = _tally(layers)
    with capsys.disabled():
        print(f"\nconfig5 layer shape (4 synthetic layers): {differing} of {elements} center "
              f"elements differ (largest difference {worst} FP16 step{'s' if worst != 1 else ''})")
    assert worst <= 1
    assert differing <= elements // 500
