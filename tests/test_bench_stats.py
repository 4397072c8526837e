"""CPU checks of bench.py's reporting helpers (no GPU): the reference
summariser's quantile and seed bootstrap
(scripts/summarize_page_gauge_results.py:24-41), the percentile summary, the
committed-traffic reader and the one-GPU guard."""

from __future__ import annotations

import random
import statistics

import numpy as np
import pytest

import bench


def test_quantile_is_numpy_linear_interpolation():
    rng = np.random.default_rng(7)
    for n in (1, 2, 5, 20, 101):
        values = rng.normal(size=n).tolist()
        for q in (0.0, 0.025, 0.25, 0.5, 0.975, 1.0):
            assert bench._quantile(values, q) == pytest.approx(np.quantile(values, q), rel=0, abs=1e-12)


def test_quantile_closed_forms():
    assert bench._quantile([4.0, 1.0, 3.0, 2.0], 0.5) == 2.5
    assert bench._quantile([1.0, 2.0], 0.025) == pytest.approx(1.025)
    assert bench._quantile([5.0], 0.975) == 5.0


def test_bootstrap_interval_is_seeded_and_bracketed():
    values = [1.61, 1.59, 1.60, 1.62, 1.597]
    first = bench.bootstrap_median_ci(values, samples=2000)
    assert first == bench.bootstrap_median_ci(values, samples=2000)
    assert min(values) <= first[0] <= statistics.median(values) <= first[1] <= max(values)
    assert bench.bootstrap_median_ci([1.5] * 5, samples=500) == [1.5, 1.5]


def test_bootstrap_matches_a_direct_resampling():
    values = [3.0, 1.0, 2.0, 5.0]
    rng = random.Random(11)
    medians = sorted(statistics.median(rng.choices(values, k=4)) for _ in range(400))
    want = [float(np.quantile(medians, 0.025)), float(np.quantile(medians, 0.975))]
    got = bench.bootstrap_median_ci(values, samples=400, seed=11)
    assert got == [round(want[0], 4), round(want[1], 4)]


def test_summarize_percentiles():
    s = bench.summarize([float(x) for x in range(1, 101)])    # ms
    assert s["p50_us"] == 50500.0 and s["min_us"] == 1000.0 and s["samples"] == 100
    assert s["p05_us"] == 6000.0 and s["p95_us"] == 95000.0


def test_committed_traffic_reads_the_profile_line():
    traffic = bench.committed_traffic(bench.ROOT)
    assert isinstance(traffic, int) and 100_000_000 < traffic < 110_000_000


def test_more_than_one_gpu_is_refused(monkeypatch, capsys):
    monkeypatch.setattr("sys.argv", ["bench.py", "--gpus", "2"])
    assert bench.main() == 2
    assert "one GPU" in capsys.readouterr().err
