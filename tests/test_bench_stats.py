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


def test_frozen_selection_takes_each_methods_argmin():
    """--pilot --freeze-splits: per shape and method the argmin split of the
    pilot's cold call p50 (the reference's FROZEN_SELECTION.json)."""
    pilot = {"splits": [0, 8, 28], "state": "cold",
             "b1_49k": {"lengths": [49152],
                        "int8": {"0": {"call_p50_us": 27.1, "items": 112},
                                 "8": {"call_p50_us": 30.0, "items": 384},
                                 "28": {"call_p50_us": 26.9, "items": 112},
                                 "argmin": "28", "planner_over_argmin": 1.007},
                        "fp16": {"0": {"call_p50_us": 42.0, "items": 112},
                                 "8": {"call_p50_us": 50.0, "items": 384},
                                 "28": {"call_p50_us": 44.0, "items": 112},
                                 "argmin": "0", "planner_over_argmin": 1.0}}}
    frozen = bench.frozen_selection(pilot)
    assert frozen["shapes"]["b1_49k"]["int8"] == 28
    assert frozen["shapes"]["b1_49k"]["fp16"] == 0
    assert frozen["shapes"]["b1_49k"]["rows"]["int8"] == {"0": 27.1, "8": 30.0, "28": 26.9}
    assert frozen["selection_timing_mode"] == "cache_neutral"


def test_trace_summary_phases_per_xcd():
    """bench.py --trace's arithmetic on two hand-made rows: one INT8 wave per
    XCD whose clocks differ by 1000 ticks (times are taken per XCD), two
    4-page groups, and the 32-bit wrap of s_memrealtime."""
    rows = np.zeros((2, 64), dtype=np.int64)
    for w, (xcc, base) in enumerate(((0, 2 ** 32 - 50), (1, 1000))):
        r = rows[w]
        r[bench.TRACE_XCC], r[bench.TRACE_KIND], r[bench.TRACE_PAGES] = xcc, 0, 8
        marks = {bench.TRACE_START: 0, bench.TRACE_IDS: 150, bench.TRACE_ISSUED: 270,
                 bench.TRACE_K: 530, bench.TRACE_V: 580, bench.TRACE_DONE: 600,
                 bench.TRACE_K + 1: 700, bench.TRACE_V + 1: 750, bench.TRACE_DONE + 1: 770,
                 bench.TRACE_END: 800}
        for lane, t in marks.items():
            r[lane] = (base + t) % 2 ** 32
    out = bench.trace_summary([rows.astype(np.uint32).view(np.int32)], [9.0])
    tick = bench.TRACE_TICK_US
    assert out["start_at"]["max"] == 0.0                       # per XCD, not across
    assert out["ids_rtt"]["p50"] == pytest.approx(150 * tick)
    assert out["first_k_after_issue"]["p50"] == pytest.approx(260 * tick)
    assert out["k_wait"]["p50"] == pytest.approx(100 * tick)   # K[1] - done[0]
    assert out["qk_to_v"]["p50"] == pytest.approx(50 * tick)
    assert out["pv"]["p50"] == pytest.approx(20 * tick)
    assert out["group_span"]["p50"] == pytest.approx(170 * tick)
    assert out["end_at"]["max"] == pytest.approx(800 * tick)
    assert out["end_at_p50_by_xcc"] == {0: 8.0, 1: 8.0}
    assert out["waves_per_call"] == 2 and out["kernel_event_mean_us"] == 9.0


def test_combine_trace_summary_boundary_per_xcd():
    """The combine rows' arithmetic: per XCD, the boundary is the first
    combine start minus the last partial end on that XCD (clocks of two
    XCDs 5000 ticks apart), the sums and the end after them only from the
    wave that writes the output (its sums mark is set)."""
    partial = np.zeros((2, 64), dtype=np.int64)
    combine = np.zeros((3, 64), dtype=np.int64)
    for w, (xcc, base) in enumerate(((0, 0), (1, 5000))):
        partial[w, bench.TRACE_XCC], partial[w, bench.TRACE_KIND] = xcc, 0
        partial[w, bench.TRACE_START], partial[w, bench.TRACE_END] = base, base + 2000
    for w, (xcc, base, sums) in enumerate(((0, 0, 2310), (0, 0, 0), (1, 5000, 2330))):
        r = combine[w]
        r[bench.TRACE_XCC], r[bench.TRACE_KIND] = xcc, bench.CTRACE_KIND
        marks = {bench.TRACE_START: 2100, bench.CTRACE_META: 2200, bench.CTRACE_ROWS: 2250,
                 bench.CTRACE_MAX: 2280, bench.CTRACE_END: 2400}
        for lane, t in marks.items():
            r[lane] = base + t
        r[bench.CTRACE_SUMS] = base + sums if sums else 0
    out = bench.combine_trace_summary([partial.astype(np.int32)], [combine.astype(np.int32)])
    tick = bench.TRACE_TICK_US
    assert out["boundary"]["p50"] == pytest.approx(100 * tick) and out["boundary"]["n"] == 2
    assert out["meta_rtt"]["p50"] == pytest.approx(100 * tick)
    assert out["rows_rtt"]["p50"] == pytest.approx(150 * tick)
    assert out["max_after_rows"]["p50"] == pytest.approx(30 * tick)
    assert out["sums_after_max"]["n"] == 2
    assert out["sums_after_max"]["max"] == pytest.approx(50 * tick)
    assert out["end_after_sums"]["p50"] == pytest.approx(80 * tick)   # 90 and 70 ticks
    assert out["end_after_sums"]["max"] == pytest.approx(90 * tick)
    assert out["wave_life"]["max"] == pytest.approx(300 * tick)
    assert out["span"]["n"] == 2


def test_combine_trace_summary_refuses_missing_rows():
    partial = np.zeros((1, 64), dtype=np.int32)
    combine = np.zeros((1, 64), dtype=np.int32)
    with pytest.raises(RuntimeError, match="combine trace rows missing"):
        bench.combine_trace_summary([partial], [combine])
