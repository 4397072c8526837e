#!/usr/bin/env python3
"""Benchmark of the PageGauge INT8 paged decode on one MI355X.

Metric: B1/49K INT8 paged-decode microseconds per call and the
fraction of the HBM roofline.  Workload: one request of 49152 tokens (3056
INT8 page-affine pages + a 256-token FP16 exact tail), Mistral-7B layer shape
(32 query / 8 KV heads, head_dim 128, 16-token pages), seeded N(0,1) K/V with
x8 on 4 of 128 channels, randomly permuted physical page table.

A step is one decode call (``pg_decode_run``): the INT8+tail split-KV partial
kernel and the combine kernel (value center and base-2 LSE included).  Following the reference protocol
(scripts/benchmark_flashinfer_page_affine_int8.py:295-349, :651-655) each
cold sample is preceded by an untimed scrub.  The reference scrubs with a
256 MiB read-modify-write; on MI355X that leaves the 256 MB Infinity Cache
full of dirty lines whose write-back then lands inside the timed call, so the
primary cold state uses a read-only 1 GiB scrub (clean eviction) and the
reference scrub is reported beside it.  Hot samples run back to back.  HIP
events on the launch stream bracket the whole call; the partial kernel (the
roofline's dominant kernel) is timed in separate samples by events that its
own dispatch stamps (hipExtLaunchKernelGGL), the interval a kernel trace
reports.

Also reported: the same-way FP16 paged-decode kernel on an FP16 copy of the
same cache (cold, hot and by the reference's paired protocol); the HBM peak
measured on the box beside the 8 TB/s spec; the reference's fused-append
increment and inclusive speedup over five validation seeds with bootstrap
intervals; configs 1, 3, 4 and 5; and the CPU baseline: the torch-CPU
restatement (oracle/cpu_baseline.py) on every host thread, for the bench
workload and the other configs.  ``--pilot`` runs the reference's split pilot
sweep instead.  Prints one JSON line.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100, help="timed cold decode calls")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--seed", type=int, default=20260840)
    p.add_argument("--scrub-mib", type=int, default=256)
    p.add_argument("--big-scrub-mib", type=int, default=1024)
    p.add_argument("--hot-repeats", type=int, default=200)
    p.add_argument("--split", type=int, default=0, help="pages per work item (0 = scheduler)")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-fp16", action="store_true")
    p.add_argument("--no-configs", action="store_true",
                   help="skip the config-1/3 decode lines and the config-4 update timing")
    p.add_argument("--sweep", default="", help="comma list of split sizes to time (pilot sweep)")
    p.add_argument("--no-decoder", action="store_true", help="skip the config-5 decoder line")
    p.add_argument("--paper-only", action="store_true",
                   help="print only the reference paper's B4 x 20K isolated-attention line")
    p.add_argument("--decoder-only", action="store_true",
                   help="run only the config-5 decoder and print its JSON")
    p.add_argument("--decoder-repeats", type=int, default=5)
    p.add_argument("--modes", default="cold_clean,cold_rmw,hot",
                   help="cache states to time (cold_clean is required: it gives value/roofline)")
    p.add_argument("--seeds", type=int, default=5,
                   help="validation seeds of the paired INT8 / FP16 study (0 = skip)")
    p.add_argument("--pilot", action="store_true",
                   help="the reference's split pilot sweep (B1/49K, B8 ragged x3, B1 16K, B1 64K): "
                        "prints one JSON line and exits")
    p.add_argument("--stream-probe", action="store_true",
                   help="time load-only walks of the B1/49K pages in the decode kernel's own "
                        "access pattern (pg_probe_decode_walk) beside the kernel; prints one "
                        "JSON line and exits")
    p.add_argument("--library-variant", default=None,
                   help="time an alternative build (python -m pagegauge_amd.build --variant NAME) "
                        "instead of the product library; the JSON line names it")
    p.add_argument("--trace", default="",
                   help="per-wave phase trace of the partial kernel from a trace build "
                        "(python -m pagegauge_amd.build --variant trace, or "
                        "trace_conditional_scales): the variant name; B1/49K, 16K and 4K, "
                        "cold calls; prints one JSON line")
    p.add_argument("--trace-calls", type=int, default=20)
    p.add_argument("--trace-dump", default="",
                   help="with --trace: also save every traced call's raw rows (partial and "
                        "combine kernels) to this .npz file, one array per workload")
    p.add_argument("--workload", choices=("b1_49k", "b1_16k", "config1", "serving_b256"),
                   default="b1_49k",
                   help="workload of the --pmc-calls driver (config1: B=1, 4096 tokens; "
                        "serving_b256: 256 ragged requests)")
    p.add_argument("--pmc-calls", type=int, default=0,
                   help="counter-collection driver for rocprofv3 --pmc: N cold decode calls, "
                        "then N plain 64 MiB copies of known size; prints one JSON line, no timing")
    p.add_argument("--freeze-splits", default="",
                   help="with --pilot: write the per-shape, per-method argmin splits to this JSON "
                        "file (the reference's FROZEN_SELECTION.json)")
    p.add_argument("--frozen-splits", default="",
                   help="a --freeze-splits file: the validation-seed study plans INT8 and FP16 "
                        "with their frozen B1/49K splits instead of the planner")
    p.add_argument("--pmc-fp16", action="store_true",
                   help="the --pmc-calls driver runs the FP16 same-way call instead of the INT8 "
                        "one (same workload, an FP16 copy of every page)")
    return p.parse_args()


def build_sources():
    """Per-source extra compiler flags of the library (pagegauge_amd.build)."""
    from pagegauge_amd import build
    return build.SOURCES


def summarize(values_ms):
    ordered = sorted(values_ms)
    n = len(ordered)
    return {
        "p50_us": 1e3 * statistics.median(ordered),
        "p05_us": 1e3 * ordered[round(0.05 * (n - 1))],
        "p95_us": 1e3 * ordered[round(0.95 * (n - 1))],
        "mean_us": 1e3 * statistics.fmean(ordered),
        "min_us": 1e3 * ordered[0],
        "samples": n,
    }


def call_samples(torch, bound, n, scrub=None):
    """Whole-call durations (ms): events recorded on the launch stream before
    and after the call, plain launches.
    ``scrub`` runs before every sample, outside the events; it also keeps the
    GPU busy while the host queues the timed launches."""
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(n)]
    for i in range(n):
        if scrub is not None:
            scrub()
        ev[i][0].record()
        bound()
        ev[i][1].record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def kernel_samples(torch, bound, n, scrub=None):
    """Partial-kernel durations (ms) from two events that the kernel's
    dispatch stamps itself (hipExtLaunchKernelGGL begin/end timestamps: the
    interval a kernel trace reports, without the launch gap).  Taken in
    separate samples because stamping the dispatch delays the call."""
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(n)]
    for row in ev:                     # a torch event has a handle once recorded
        for e in row:
            e.record()
    torch.cuda.synchronize()
    for i in range(n):
        if scrub is not None:
            scrub()
        bound.partial_timed(ev[i][0].cuda_event, ev[i][1].cuda_event)
        bound.combine()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def graph_call_samples(torch, bind, n, scrub):
    """Whole-call durations (ms) of the call captured in a HIP graph and
    replayed, the way the decoder's step graphs run the partial and combine
    kernels.  ``bind(stream)`` returns the call bound to the capture stream;
    the replay runs on the current stream between the two events, after the
    untimed ``scrub``."""
    stream = torch.cuda.Stream()
    bound = bind(stream.cuda_stream)
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        bound()                                    # eager warm-up on the capture stream
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        bound()
    torch.cuda.synchronize()
    for _ in range(3):
        scrub()
        graph.replay()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(n)]
    for i in range(n):
        scrub()
        ev[i][0].record()
        graph.replay()
        ev[i][1].record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def graph_fixed_cost(torch, scrub, n: int = 40):
    """Event-to-event p50 (µs) of one 1-element fill kernel launched eagerly
    and as a one-node HIP graph, after the same untimed scrub: the cost a
    graph replay adds independently of what it holds."""
    tiny = torch.zeros(1, device=torch.cuda.current_device())
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        tiny.zero_()
    torch.cuda.synchronize()
    result = {}
    for name, fn in (("eager_fill_p50_us", tiny.zero_), ("graph_fill_p50_us", graph.replay)):
        for _ in range(3):
            scrub()
            fn()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(n)]
        for i in range(n):
            scrub()
            ev[i][0].record()
            fn()
            ev[i][1].record()
        torch.cuda.synchronize()
        result[name] = round(1e3 * statistics.median([a.elapsed_time(b) for a, b in ev]), 3)
    return result


def timed_calls(torch, bound, n, scrub=None):
    """(partial kernel ms list, whole call ms list), n samples of each."""
    call = call_samples(torch, bound, n, scrub)
    kernel = kernel_samples(torch, bound, n, scrub)
    return kernel, call


def measure(torch, bound, args, scrub_clean, scrub_rmw):
    """Three cache states: cold-clean (read-only 1 GiB scrub: MALL holds no
    line of the cache and no dirty line), cold-rmw (the reference's 256 MiB
    add_ scrub, which also leaves up to 256 MB of dirty lines whose
    write-back lands inside the timed call) and hot (back to back)."""
    modes = set(args.modes.split(","))
    for _ in range(args.warmup):
        scrub_clean()
        bound()
    torch.cuda.synchronize()
    cold_k, cold_c = timed_calls(torch, bound, args.steps, scrub=scrub_clean)
    result = {"cold_clean_1gib": {"kernel": summarize(cold_k), "call": summarize(cold_c)},
              "_cold_kernel_ms": cold_k, "_cold_call_ms": cold_c}
    if "cold_rmw" in modes:
        rmw_k, rmw_c = timed_calls(torch, bound, max(10, args.steps // 2), scrub=scrub_rmw)
        result["cold_rmw_256mib"] = {"kernel": summarize(rmw_k), "call": summarize(rmw_c)}
    if "hot" not in modes:
        return result
    # hot: back-to-back calls (no events in between) after a long head-start
    # kernel; per-call time = span / repeats
    hot = []
    for _ in range(5):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        scrub_clean()
        bound()
        start.record()
        for _ in range(args.hot_repeats):
            bound()
        end.record()
        torch.cuda.synchronize()
        hot.append(start.elapsed_time(end) / args.hot_repeats)
    result["hot"] = {"call": summarize(hot), "repeats_per_sample": args.hot_repeats}
    return result


def controlled_pair(torch, operations: dict, warmup: int, repeats: int, scrub):
    """The reference's paired protocol (controlled_event_times,
    scripts/benchmark_flashinfer_page_affine_int8.py:295-349) for two
    methods: in each repeat both run, in A/B then B/A order alternately;
    every cache-neutral sample follows a scrub and every cache-hot sample
    an untimed call of the same method; events bracket the call only.
    Returns per mode the p50/mean of each method and the p50 ratio B/A."""
    names = list(operations)
    out = {}
    for mode in ("cache_neutral", "cache_hot"):
        events = {name: [] for name in names}
        for repeat in range(warmup + repeats):
            for name in (names if repeat % 2 == 0 else names[::-1]):
                if mode == "cache_neutral":
                    scrub()
                else:
                    operations[name]()
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record()
                operations[name]()
                end.record()
                if repeat >= warmup:
                    events[name].append((start, end))
        torch.cuda.synchronize()
        row = {name: summarize([a.elapsed_time(b) for a, b in pairs])
               for name, pairs in events.items()}
        row["ratio_p50"] = round(row[names[1]]["p50_us"] / row[names[0]]["p50_us"], 4)
        out[mode] = row
    return out


def pmc_driver(torch, bound, calls, scrub_clean, device):
    """Workload for one ``rocprofv3 --pmc`` pass (no timing): ``calls`` cold
    decode calls, then ``calls`` plain copies of 64 MiB (64 MiB read + 64 MiB
    written, the known-size reference that calibrates FETCH_SIZE/WRITE_SIZE)."""
    src = torch.ones(64 << 18, dtype=torch.int32, device=device)
    dst = torch.empty_like(src)
    for _ in range(calls):
        scrub_clean()
        bound()
    for _ in range(calls):
        scrub_clean()
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"pmc_calls": calls, "copy_bytes": src.numel() * 4}


def committed_traffic(root: Path):
    """HBM bytes per launch of the partial kernel from the committed counter
    summary (two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by
    the plain-copy calibration), or None."""
    path = root / "profiles" / "decode_partial_b1_49k_pmc.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def decode_config(torch, decode, w, scrub, samples: int):
    """Cold (clean-scrub) call p50 and partial-kernel mean of one workload."""
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=w.query.device)
    out = torch.empty_like(w.query)
    lse = torch.empty(w.batch, 32, dtype=torch.float32, device=w.query.device)
    dec = decode.PageGaugeSegmentedDecode(ws)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len)
    bound = dec.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                     (w.tail_k, w.tail_v), w.value_center, out=out, lse=lse)
    for _ in range(3):
        scrub()
        bound()
    kernel, call = timed_calls(torch, bound, samples, scrub=scrub)
    graph = graph_call_samples(
        torch, lambda s: dec.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                                  (w.tail_k, w.tail_v), w.value_center, out=out, lse=lse,
                                  stream=s), samples, scrub)
    kernel_us = 1e3 * statistics.fmean(kernel)
    alg = w.algorithmic_bytes()
    res = {
        "lengths": w.lengths if len(w.lengths) <= 8 else len(w.lengths),
        "work_items": dec.num_work_items,
        "call_p50_us": round(1e3 * statistics.median(call), 3),
        "graph_call_p50_us": round(1e3 * statistics.median(graph), 3),
        "kernel_mean_us": round(kernel_us, 3),
        "algorithmic_bytes": alg,
        "achieved_gbps": round(alg / (kernel_us * 1e-6) / 1e9, 1),
        "frac_of_peak": round(alg / (kernel_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
    }
    if w.fp16_k is not None:
        # the same-way FP16 kernel over an FP16 copy of every page, timed alike
        wrap16 = decode.BatchDecodeWithPagedKVCacheWrapper(
            torch.empty(64 << 20, dtype=torch.uint8, device=w.query.device), "NHD")
        wrap16.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 32, 8, 128, 16,
                    kv_data_type=torch.float16)
        b16 = wrap16.bind(w.query, (w.fp16_k, w.fp16_v), out=torch.empty_like(w.query),
                          lse=torch.empty_like(lse))
        for _ in range(3):
            scrub()
            b16()
        call16 = call_samples(torch, b16, samples, scrub)
        res["fp16_same_way_call_p50_us"] = round(1e3 * statistics.median(call16), 3)
        res["speedup_vs_fp16_same_way"] = round(statistics.median(call16) / statistics.median(call), 4)
    return res


# The reference paper's isolated-attention microbenchmark on RTX 5090
# (paper/mlsys2027/main.tex:140-156): B=4, 20,481-token contexts, mean latency
# over 120 repeats with 256 MiB cache scrubs.
PAPER_B4_20K_RTX5090_US = {"segmented": 132.20, "heterogeneous": 143.06, "fp16": 220.75}


def heterogeneous_call(torch, decode, w, device, out):
    """The heterogeneous one-table decode of workload ``w`` as a callable
    writing ``out``: one unified table per request (its INT8 pages, then its
    FP16 ring pages, ``old_kv_len`` = the INT8 tokens), planned with the
    exact-tail hint of the ring's 16 pages."""
    old_ptr, tail_ptr = w.old_indptr.tolist(), w.tail_indptr.tolist()
    old_idx, tail_idx = w.old_indices.cpu(), w.tail_indices.cpu()
    rows, indptr, old_len = [], [0], []
    for b in range(w.batch):
        rows += [old_idx[old_ptr[b]:old_ptr[b + 1]], tail_idx[tail_ptr[b]:tail_ptr[b + 1]]]
        indptr.append(indptr[-1] + old_ptr[b + 1] - old_ptr[b] + tail_ptr[b + 1] - tail_ptr[b])
        old_len.append(16 * (old_ptr[b + 1] - old_ptr[b]))
    unified = torch.cat(rows).to(device)
    old_kv_len = torch.tensor(old_len, dtype=torch.int32, device=device)
    het = decode.make_heterogeneous_page_gauge_wrapper(
        None, torch.empty(64 << 20, dtype=torch.uint8, device=device))
    het.plan(torch.tensor(indptr, dtype=torch.int32), unified, w.tail_last_page_len, 32, 8, 128, 16,
             exact_tail_pages_hint=16)
    args = (w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, w.tail_k, w.tail_v,
            old_kv_len, w.value_center)
    het.run(*args, out=out)                      # validates once
    call = lambda: het.run(*args, out=out)       # noqa: E731
    call.keep = (het, unified, old_kv_len)       # tables and workspace outlive the callable's use
    return call


def paper_b4_20k(torch, decode, workloads, device, scrub, samples: int):
    """The paper's B4 x 20K isolated-attention shape on this GPU: four
    requests of 20480 tokens (1264 INT8 + 16 FP16 pages each; the paper's
    20,481st token would add one row to a 1281st page), each call cold after
    the 1 GiB read scrub.  Segmented call (partial + combine), heterogeneous
    one-table call (the same pages through one unified table per request)
    and the FP16 same-way kernel over an all-FP16 copy; mean and p50 of the
    whole call, beside the paper's RTX 5090 means."""
    w = workloads.build_decode_workload([20480] * 4, workloads.VALIDATION_SEEDS[0], device=device,
                                        with_fp16_copy=True)
    out = torch.empty_like(w.query)
    lse = torch.empty(w.batch, 32, dtype=torch.float32, device=device)
    bounds = {}
    seg = decode.PageGaugeSegmentedDecode(torch.empty(64 << 20, dtype=torch.uint8, device=device))
    seg.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len)
    bounds["segmented"] = seg.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                                   (w.tail_k, w.tail_v), w.value_center, out=out, lse=lse)
    out_h = torch.empty_like(w.query)
    bounds["heterogeneous"] = heterogeneous_call(torch, decode, w, device, out_h)
    fp16 = decode.BatchDecodeWithPagedKVCacheWrapper(
        torch.empty(64 << 20, dtype=torch.uint8, device=device), "NHD")
    fp16.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 32, 8, 128, 16,
              kv_data_type=torch.float16)
    out16 = torch.empty_like(w.query)
    bounds["fp16"] = fp16.bind(w.query, (w.fp16_k, w.fp16_v), out=out16, lse=torch.empty_like(lse))
    res = {"lengths": w.lengths, "algorithmic_bytes": {"page_gauge": w.algorithmic_bytes(),
                                                       "fp16": w.fp16_algorithmic_bytes()}}
    for name, call in bounds.items():
        for _ in range(3):
            scrub()
            call()
        ms = call_samples(torch, call, samples, scrub)
        mean_us = 1e3 * statistics.fmean(ms)
        res[name] = {"call_mean_us": round(mean_us, 2),
                     "call_p50_us": round(1e3 * statistics.median(ms), 2),
                     "rtx5090_paper_mean_us": PAPER_B4_20K_RTX5090_US[name],
                     "rtx5090_over_this": round(PAPER_B4_20K_RTX5090_US[name] / mean_us, 2)}
    torch.cuda.synchronize()
    res["heterogeneous_vs_segmented_max_abs"] = float((out_h.float() - out.float()).abs().max())
    res["fp16_over_segmented"] = round(res["fp16"]["call_mean_us"] / res["segmented"]["call_mean_us"],
                                       3)
    return res


# The reference paper's full-decoder measurement (paper/mlsys2027/main.tex:277):
# Mistral-7B, B=4, context 20480, CUDA graphs, RTX 5090.
PAPER_B4_20K_DECODER_RTX5090 = {"page_gauge": {"ms_per_step": 15.16, "tokens_per_s": 263.9},
                                "fp16": {"ms_per_step": 17.05, "tokens_per_s": 234.7}}


def decoder_b4_20k(torch, device, repeats: int):
    """The paper's B4 x 20480 full-decoder shape on this GPU (the config-5
    decoder with four requests in lockstep), beside the paper's RTX 5090
    numbers.  Not the same run: random-init weights of the same architecture
    (the same bytes and kernels), 16 greedy steps instead of 512
    teacher-forced ones, and this build's 256-token exact tail instead of the
    paper's 768-token tail with 4 sink and 128 static-suffix exact pages.
    A timing line: the logit gate is config 5's (random-init weights give
    near-flat logits, so all-four-requests top-1 agreement says little)."""
    res = decoder_config5(torch, device, repeats, context=20480, steps=16, batch=4,
                          logit_gate=False)
    res["rtx5090_paper"] = PAPER_B4_20K_DECODER_RTX5090
    for name in ("page_gauge", "fp16"):
        res[name]["rtx5090_paper_over_this"] = round(
            PAPER_B4_20K_DECODER_RTX5090[name]["ms_per_step"] / res[name]["ms_per_token_wall_p50"], 2)
    return res


def config4_inputs(torch):
    """Seeded config-4 inputs on the CPU (seed 20260840): start lengths, RoPE
    tables (theta 1e6), per-request centers and 16 steps of q/k/v."""
    from pagegauge_amd import decoder

    gen = torch.Generator().manual_seed(20260840)
    start = [4096, 4099, 8192, 8199, 12288, 12299, 16384, 16398]
    batch, steps = 8, 16
    cos, sin = decoder.rope_tables(max(start) + steps, 1.0e6)
    rnd = lambda *shape, s=1.0: (torch.randn(*shape, generator=gen) * s).half()  # noqa: E731
    kc, vc = rnd(batch, 8, 128, s=0.1), rnd(batch, 8, 128, s=0.1)
    return {"start": start, "cos": cos, "sin": sin, "key_center": kc, "value_center": vc,
            "q": [rnd(batch, 32, 128) for _ in range(steps)],
            "k": [rnd(batch, 8, 128) for _ in range(steps)],
            "v": [rnd(batch, 8, 128) for _ in range(steps)], "generator": gen}


def exact_tail_merge_line(torch, device, scrub, samples: int = 40):
    """The reference's fused exact-tail merge (``exact_tail_merge_center``,
    tests/page_gauge_append_extension.cu:389-583) over full 16-page tails at
    B = 1 and 8: cold p50 of the call (events around it, after the clean
    scrub, which also covers the host's argument checks)."""
    from pagegauge_amd import runtime

    ext = runtime.load_append_extension()
    out = {}
    for batch in (1, 8):
        gen = torch.Generator().manual_seed(20260840 + batch)
        ring = 16
        q = torch.randn(batch, 32, 128, generator=gen).half().to(device)
        ek = (torch.randn(batch * ring, 16, 8, 128, generator=gen) * 0.35).half().to(device)
        ev = (torch.randn(batch * ring, 16, 8, 128, generator=gen) * 0.35).half().to(device)
        center = (torch.randn(batch, 8, 128, generator=gen) * 0.1).half().to(device)
        idx = torch.randperm(batch * ring, generator=gen).to(torch.int32).to(device)
        last = torch.full((batch,), 16, dtype=torch.int32, device=device)
        old = torch.randn(batch, 32, 128, generator=gen).half().to(device)
        lse = (torch.randn(batch, 32, generator=gen) + 8).float().to(device)

        def call():
            ext.exact_tail_merge_center(q, ek, ev, idx, last, old, lse,
                                        center if batch > 1 else center[0], 128 ** -0.5)

        for _ in range(3):
            scrub()
            call()
        out[f"b{batch}"] = {"tail_pages": ring,
                            "cold_call": summarize(call_samples(torch, call, samples, scrub))}
    return out


def update_config4(torch, device, replays: int):
    """Config 4 cache update: B=8, 16 decode steps (start lengths
    4096, 4099, ..., 16398: every row closes one page, four of them mid-window),
    RoPE theta 1e6 at position = current length.  The 16 steps are captured in
    a HIP graph and replayed back to back; reported as GPU µs per step for the
    fused RoPE + centered append + finalize kernel (per-request positions),
    the centered append + finalize without RoPE, and the plain FP16 append
    (the reference's incremental-cost baseline,
    scripts/benchmark_page_gauge_overheads.py:86-205)."""
    from pagegauge_amd import runtime, update

    ext = runtime.load_append_extension()
    inputs = config4_inputs(torch)
    start, batch, ring, steps = inputs["start"], 8, 16, 16
    code_pages = (max(start) + steps + 15) // 16
    cos, sin = inputs["cos"].to(device), inputs["sin"].to(device)
    kc, vc = inputs["key_center"].to(device), inputs["value_center"].to(device)
    kc_shared, vc_shared = kc[0].contiguous(), vc[0].contiguous()
    q = [t.to(device) for t in inputs["q"]]
    k = [t.to(device) for t in inputs["k"]]
    v = [t.to(device) for t in inputs["v"]]
    gen = inputs["generator"]
    rnd = lambda *shape, s=1.0: (torch.randn(*shape, generator=gen) * s).half().to(device)  # noqa: E731
    pos = [torch.tensor([x + t for x in start], dtype=torch.int32, device=device) for t in range(steps)]
    # per-request (page id, offset) of a request-major FP16 / exact pool
    page_ids = [torch.tensor([r * code_pages + (x + t) // 16 for r, x in enumerate(start)],
                             dtype=torch.int32, device=device) for t in range(steps)]
    offsets = [torch.tensor([(x + t) % 16 for x in start], dtype=torch.int32, device=device)
               for t in range(steps)]
    exact = [rnd(batch * ring, 16, 8, 128) for _ in range(2)]
    codes = [torch.zeros(batch * code_pages, 16, 8, 128, dtype=torch.int8, device=device) for _ in range(2)]
    scales = [torch.zeros(batch * code_pages, 8, dtype=torch.float16, device=device) for _ in range(2)]
    pool = [rnd(batch * code_pages, 16, 8, 128) for _ in range(2)]
    rq = torch.zeros(batch, 32, 128, dtype=torch.float16, device=device)

    def fused():
        for t in range(steps):
            ext.rope_append_page_gauge_positions(q[t], k[t], v[t], cos, sin, pos[t], kc, vc, rq,
                                                 exact[0], exact[1], codes[0], codes[1],
                                                 scales[0], scales[1], 0)

    def finalize():
        for t in range(steps):
            update.append_finalize_page_gauge(k[t], v[t], kc_shared, vc_shared, pool[0], pool[1],
                                              codes[0], codes[1], scales[0], scales[1],
                                              page_ids[t], offsets[t])

    def fp16():
        for t in range(steps):
            update.append_kv(k[t], v[t], pool[0], pool[1], page_ids[t], offsets[t])

    result = {"batch": batch, "steps_per_graph": steps, "replays": replays,
              "closing_rows_per_window": 8}
    stream = torch.cuda.Stream()
    for name, fn in (("fused_rope_append_finalize", fused), ("append_finalize", finalize),
                     ("fp16_append", fp16)):
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            fn()                                   # eager warm-up on the capture stream
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            fn()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        result[name + "_us_per_step"] = round(1e3 * e0.elapsed_time(e1) / (replays * steps), 3)
    result["incremental_us_per_step"] = round(result["append_finalize_us_per_step"] -
                                              result["fp16_append_us_per_step"], 3)
    return result


def decoder_config5(torch, device, repeats: int, context: int = 16384, steps: int = 16,
                    seed: int = 20260850, batch: int = 1, logit_gate: bool = True):
    """Config 5: random-init Mistral-7B-shaped decoder, ``batch`` requests
    (B=1 for config 5), ``context``-token prefills of uniform random ids, then
    ``steps`` greedy decode steps with every layer on the INT8 paged KV + FP16
    tail (K2 append + K1 decode), each step one HIP graph.  Reports ms per
    step (= ms/token at B=1) and tokens/s of the PageGauge decoder and of the
    same decoder over an FP16 cache, and the reference's logit gate
    (cosine >= 0.995, top-1 agreement, max-abs;
    scripts/benchmark_page_gauge_transformer.py:3865-3903) on a teacher-forced
    sequence of random tokens (``logit_gate``)."""
    import torch.nn.functional as F

    from pagegauge_amd import decoder as dec

    t0 = time.perf_counter()
    cfg = dec.DecoderConfig()
    weights = dec.DecoderWeights(cfg, seed, device=device)
    torch.cuda.synchronize()                   # the weight fill runs on the GPU
    gen = torch.Generator().manual_seed(seed)
    if batch == 1:
        prompt = torch.randint(0, cfg.vocab, (context,), generator=gen)
        forced = torch.randint(0, cfg.vocab, (steps, 1), generator=gen).to(device)
    else:
        prompt = torch.randint(0, cfg.vocab, (batch, context), generator=gen)
        forced = torch.randint(0, cfg.vocab, (steps, batch), generator=gen).to(device)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    first, _, decoders = dec.build_decoders(weights, prompt, steps + 1)
    base = decoders["page_gauge"]
    # the one-launch unified-table variant (a12) over a copy of the same cache
    decoders["page_gauge_heterogeneous"] = dec.PageGaugeDecoder(
        weights, base.cache.clone(), "page_gauge", base.max_pages * 16, base.rope_cos,
        base.rope_sin, batch_size=batch, tail_attention="heterogeneous")
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    result = {"model": "Mistral-7B architecture, random-init fp16 (32 layers, hidden 4096, "
                       "32/8 heads, MLP 14336, vocab 32768)",
              "batch": batch, "prefill_tokens": context, "decode_steps": steps, "repeats": repeats,
              "weights_init_s": round(t1 - t0, 2), "prefill_and_cache_build_s": round(t2 - t1, 2)}
    kv_bytes = {}
    per_layer_pages = math.ceil((context + steps) / 16)
    kv_bytes["page_gauge"] = cfg.layers * ((per_layer_pages - 16) * (2 * 16 * 8 * 128 + 4 * 8)
                                           + 16 * 2 * 16 * 8 * 256 + 2 * 8 * 128 * 2)
    kv_bytes["fp16"] = cfg.layers * per_layer_pages * 2 * 16 * 8 * 256
    kv_bytes["page_gauge_heterogeneous"] = kv_bytes["page_gauge"]
    weight_bytes = weights.bytes_per_token()
    logits = {}
    names = list(decoders)
    for d in decoders.values():
        d.generate(first, context, steps, use_graphs=True)          # capture + warm
    torch.cuda.synchronize()
    walls = {name: [] for name in names}
    gpu = {name: [] for name in names}
    tokens_ref = {}
    # the decoders take turns, in a rotating order, so that a drift of the
    # GPU's clocks or caches over the run does not favour one of them
    for rep in range(repeats):
        for k in range(len(names)):
            name = names[(rep + k) % len(names)]
            d = decoders[name]
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            e0.record()
            toks, _ = d.generate(first, context, steps, use_graphs=True)
            e1.record()
            torch.cuda.synchronize()
            walls[name].append(time.perf_counter() - w0)
            gpu[name].append(e0.elapsed_time(e1) * 1e-3)
            tokens_ref.setdefault(name, toks)
            if not torch.equal(toks, tokens_ref[name]):
                raise RuntimeError("greedy decode is not deterministic across repeats")
    # eager steps (no graph), timed the same way, for the launch-overhead
    # comparison
    eager = {name: [] for name in names}
    for d in decoders.values():
        d.drop_graphs()
        d.generate(first, context, steps, use_graphs=False)         # warm
    for rep in range(repeats):
        for k in range(len(names)):
            name = names[(rep + k) % len(names)]
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            toks, _ = decoders[name].generate(first, context, steps, use_graphs=False)
            torch.cuda.synchronize()
            eager[name].append(time.perf_counter() - w0)
            if not torch.equal(toks, tokens_ref[name]):
                raise RuntimeError("eager and graph greedy decodes differ")
    for name in names:
        d = decoders[name]
        eager_s = statistics.median(eager[name])
        ms_token = 1e3 * statistics.median(walls[name]) / steps          # per decode step
        total_bytes = weight_bytes + batch * kv_bytes[name]
        result[name] = {
            "ms_per_token_wall_p50": round(ms_token, 4),
            "ms_per_token_gpu_p50": round(1e3 * statistics.median(gpu[name]) / steps, 4),
            "tokens_per_s": round(batch * 1e3 / ms_token, 2),
            "eager_ms_per_token": round(1e3 * eager_s / steps, 4),
            "eager_tokens_per_s": round(batch * steps / eager_s, 2),
            "bytes_per_token": total_bytes,
            "achieved_gbps": round(total_bytes / (ms_token * 1e-3) / 1e9, 1),
            "hbm_frac": round(total_bytes / (ms_token * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "greedy_tokens": [int(t) for t in tokens_ref[name].reshape(-1).tolist()],
        }
        if logit_gate:                          # teacher-forced logits for the comparison
            logits[name] = [d.step(forced[i], context + i).clone() for i in range(steps)]
        del d
    if "page_gauge" in logits and "fp16" in logits:
        cos = [float(F.cosine_similarity(a, b, dim=-1).min())
               for a, b in zip(logits["page_gauge"], logits["fp16"])]
        top1 = [bool((a.argmax(-1) == b.argmax(-1)).all())
                for a, b in zip(logits["page_gauge"], logits["fp16"])]
        max_abs = max(float((a - b).abs().max()) for a, b in zip(logits["page_gauge"], logits["fp16"]))
        result["page_gauge_vs_fp16_logits"] = {
            "min_cosine": round(min(cos), 6), "top1_agreement": sum(top1) / len(top1),
            "max_abs": round(max_abs, 5), "gate": "cosine >= 0.995 (reference default)",
            "passed": min(cos) >= 0.995}
        result["speedup_vs_fp16_cache"] = round(result["fp16"]["ms_per_token_wall_p50"]
                                                / result["page_gauge"]["ms_per_token_wall_p50"], 4)
    del decoders, weights
    torch.cuda.empty_cache()
    return result


def _cpu_samples(fn, calls: int, warmup: int = 3):
    """Warm-up calls, then ``calls`` timed calls (time.perf_counter), in ms."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(calls):
        t0 = time.perf_counter()
        fn()
        times.append(1e3 * (time.perf_counter() - t0))
    return times


def _decode_on_host(torch, w):
    """The CPU copies of a decode workload, as ``cpu_baseline.decode_dense``
    arguments."""
    c = lambda t: t.detach().cpu()  # noqa: E731
    return dict(query=c(w.query), k_pages=c(w.k_codes), v_pages=c(w.v_codes), indptr=c(w.old_indptr),
                indices=c(w.old_indices), last_page_len=c(w.old_last_page_len), sm_scale=w.sm_scale,
                k_scale=c(w.k_scale), v_scale=c(w.v_scale), tail_k=c(w.tail_k), tail_v=c(w.tail_v),
                tail_indptr=c(w.tail_indptr), tail_indices=c(w.tail_indices),
                tail_last_page_len=c(w.tail_last_page_len), value_center=c(w.value_center))


def cpu_baseline(torch, w, device, calls: int = 20, configs: bool = True):
    """The torch-CPU restatement (oracle/cpu_baseline.py) on every host
    thread, in this process, on the same seeded inputs as the GPU lines:
    3 warm-ups then ``calls`` timed calls per config (p05/p50/p95 ms).
    B1/49K is the bench workload (the ``value`` of the CPU line); config 1
    is BASELINE's primary CPU point; config 3 is its first seed; config 4 is
    one 16-step update window; config 5 is capped (2 of 32 layers, 4 decode
    steps) and also reported scaled to 32 layers."""
    from oracle import cpu_baseline as cb
    from pagegauge_amd import workloads

    torch.set_num_threads(os.cpu_count() or 1)
    host = cb.host_description()
    out = {"host": host}
    b1 = _decode_on_host(torch, w)
    result = {}
    ms = _cpu_samples(lambda: result.update(r=cb.decode_dense(**b1)), calls)
    out["b1_49k"] = {"ms": summarize(ms), "out": result["r"][0], "lse": result["r"][1]}
    if not configs:
        return out
    w1 = workloads.single_4k(workloads.VALIDATION_SEEDS[0], device=device)
    c1 = _decode_on_host(torch, w1)
    out["config1_b1_4k"] = {"ms": summarize(_cpu_samples(lambda: cb.decode_dense(**c1), calls))}
    del w1
    w3 = workloads.b8_ragged(workloads.VALIDATION_SEEDS[0], device=device)
    c3 = _decode_on_host(torch, w3)
    out["config3_b8_ragged_seed0"] = {"lengths": w3.lengths,
                                      "ms": summarize(_cpu_samples(lambda: cb.decode_dense(**c3), calls))}
    del w3, c3
    torch.cuda.empty_cache()
    inputs = config4_inputs(torch)
    start, steps, ring = inputs["start"], 16, 16
    code_pages = (max(start) + steps + 15) // 16
    state = [torch.zeros(8 * ring, 16, 8, 128, dtype=torch.float16) for _ in range(2)]
    state += [torch.zeros(8 * code_pages, 16, 8, 128, dtype=torch.int8) for _ in range(2)]
    state += [torch.zeros(8 * code_pages, 8, dtype=torch.float16) for _ in range(2)]
    rq = torch.zeros(8, 32, 128, dtype=torch.float16)
    positions = [torch.tensor([x + t for x in start], dtype=torch.int32) for t in range(steps)]

    def window():
        for t in range(steps):
            cb.append_positions(inputs["q"][t], inputs["k"][t], inputs["v"][t], inputs["cos"],
                                inputs["sin"], positions[t], inputs["key_center"],
                                inputs["value_center"], rq, *state)

    win = summarize(_cpu_samples(window, calls))
    out["config4_update"] = {"ms_per_16_step_window": win,
                             "us_per_step_p50": round(1e3 * win["p50_us"] / 1e3 / steps, 3)}
    layers, context, dsteps = 2, 16384, 4
    t0 = time.perf_counter()
    model = cb.CpuDecoder(layers, context, 20260850, steps=dsteps + 8)
    build_s = time.perf_counter() - t0
    position = [context]

    def step():
        model.step(7, position[0])
        position[0] += 1

    step_ms = _cpu_samples(step, dsteps, warmup=3)
    per_layer = statistics.median(step_ms) / layers
    out["config5_decoder_capped"] = {
        "cap": f"{layers} of 32 layers, {dsteps} timed decode steps after 3 warm-ups, 16384-token "
               f"cache of random K/V (INT8 history + 16-page ring), float32 weights",
        "ms_per_step": summarize(step_ms), "build_s": round(build_s, 2),
        "scaled_to_32_layers_ms_per_token": round(per_layer * 32, 2),
        "scaled_tokens_per_s": round(1e3 / (per_layer * 32), 3)}
    del model
    return out


def _probes():
    """bench.py's probe library (libpagegauge_bench.so, include/pagegauge_bench.h)."""
    from pagegauge_amd import _capi
    return _capi.bench_library()


def _probe_check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"probe: {_probes().pg_last_error().decode()} (code {rc})")


def measure_peak(torch, device, w, scrub, samples: int = 10):
    """HBM read bandwidth on this box, beside the 8 TB/s specification, from
    the library's read probes (pg_probe_linear_read, pg_probe_page_walk):
    a 1 GiB linear read; a cold linear read of B1/49K's algorithmic bytes
    (101,316,248 B) after ``scrub`` (the decode's clean 1 GiB read), and the
    same read hot; and a cold walk of the B1/49K INT8 pages in their permuted order,
    every page read as contiguous 16 KiB of K and of V codes (the most
    favourable way to stream this cache).  Timed like the decode kernel:
    events stamped by the probe's own dispatch, mean over ``samples``, best
    of a few launch shapes."""
    lib = _probes()
    stream = torch.cuda.current_stream().cuda_stream
    big = torch.ones((1 << 30) // 4, dtype=torch.int32, device=device)
    small = torch.ones(101316248 // 16 * 4, dtype=torch.int32, device=device)
    sink = torch.empty(1 << 16, dtype=torch.int32, device=device)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(samples)]
    for pair in events:
        for e in pair:
            e.record()
    torch.cuda.synchronize()

    def linear(t, blocks, ev=(None, None)):
        _probe_check(lib.pg_probe_linear_read(t.data_ptr(), t.numel() * 4, sink.data_ptr(),
                                              sink.numel(), blocks, ev[0], ev[1], stream))

    pages = int(w.old_indices.numel())

    def walk(per_block, ev=(None, None)):
        _probe_check(lib.pg_probe_page_walk(w.k_codes.data_ptr(), w.v_codes.data_ptr(),
                                            w.old_indices.data_ptr(), pages, per_block, 16384,
                                            sink.data_ptr(), sink.numel(), ev[0], ev[1], stream))

    def timed(fn, before=None):
        """Mean dispatch-stamped duration (s) of ``fn(events)``."""
        for _ in range(2):
            if before is not None:
                before()
            fn((None, None))
        for pair in events:
            if before is not None:
                before()
            fn((pair[0].cuda_event, pair[1].cuda_event))
        torch.cuda.synchronize()
        return statistics.fmean(a.elapsed_time(b) for a, b in events) * 1e-3

    # Cold means after ``scrub``, the decode's own clean 1 GiB read (regular
    # loads, which allocate in the Infinity Cache and so evict it).  The
    # probe's nontemporal read would not do: its loads do not allocate there,
    # and a page walk after it still finds about a third of its pages cached
    # (16.0 against 19.0 µs after the clean scrub, 14.3 µs hot).
    shapes = (256, 512, 1024, 2048)
    read_1g = min(timed(lambda ev, b=b: linear(big, b, ev)) for b in shapes)
    cold = min(timed(lambda ev, b=b: linear(small, b, ev), scrub) for b in shapes)
    hot = min(timed(lambda ev, b=b: linear(small, b, ev)) for b in shapes)
    walk_t = min(timed(lambda ev, p=p: walk(p, ev), scrub) for p in (2, 4, 8, 12))
    walk_bytes = pages * 2 * 16384
    res = {"read_1gib_gbps": round((1 << 30) / read_1g / 1e9, 1),
           "cold_read_101mb_gbps": round(small.numel() * 4 / cold / 1e9, 1),
           "cold_read_101mb_us": round(cold * 1e6, 2),
           "hot_read_101mb_gbps": round(small.numel() * 4 / hot / 1e9, 1),
           "cold_page_walk_b1_49k_gbps": round(walk_bytes / walk_t / 1e9, 1),
           "cold_page_walk_b1_49k_us": round(walk_t * 1e6, 2),
           "method": "pg_probe_linear_read / pg_probe_page_walk; events stamped by the probe's "
                     "dispatch (as the decode kernel's); best launch shape of the mean over %d; "
                     "cold = after the decode's clean 1 GiB read scrub" % samples}
    del big, small
    torch.cuda.empty_cache()
    return res


def append_overhead(torch, device, scrub, batch: int = 1, warmup: int = 3, repeats: int = 30):
    """The reference's incremental cost of the fused append + finalize
    (scripts/benchmark_page_gauge_overheads.py:522-636): 16-step cycles of
    the plain FP16 append against the centered append + finalize at the same
    per-request (page, offset), timed by the paired protocol (cache-neutral:
    a scrub before each sample; cache-hot: a same-method call before it),
    divided by 16; incremental = max(0, fused - plain) per decode step."""
    from pagegauge_amd import update

    gen = torch.Generator().manual_seed(20260840)
    shape = (batch, 16, 8, 128)
    key = [(torch.randn(batch, 8, 128, generator=gen)).half().to(device) for _ in range(16)]
    value = [(torch.randn(batch, 8, 128, generator=gen)).half().to(device) for _ in range(16)]
    kc = (torch.randn(8, 128, generator=gen) * 0.1).half().to(device)
    vc = (torch.randn(8, 128, generator=gen) * 0.1).half().to(device)
    plain = [torch.zeros(shape, dtype=torch.float16, device=device) for _ in range(2)]
    fused = [torch.zeros(shape, dtype=torch.float16, device=device) for _ in range(2)]
    fused += [torch.zeros(shape, dtype=torch.int8, device=device) for _ in range(2)]
    fused += [torch.zeros(batch, 8, dtype=torch.float16, device=device) for _ in range(2)]
    ids = torch.arange(batch, dtype=torch.int32, device=device)
    offsets = [torch.full((batch,), t, dtype=torch.int32, device=device) for t in range(16)]

    def plain_cycle():
        for t in range(16):
            update.append_kv(key[t], value[t], *plain, ids, offsets[t])

    def fused_cycle():
        for t in range(16):
            update.append_finalize_page_gauge(key[t], value[t], kc, vc, *fused, ids, offsets[t])

    pair = controlled_pair(torch, {"fp16_append_only": plain_cycle,
                                   "page_gauge_fused_append_finalize": fused_cycle},
                           warmup, repeats, scrub)
    out = {"batch": batch}
    for mode in ("cache_neutral", "cache_hot"):
        a = pair[mode]["fp16_append_only"]["p50_us"] / 16
        b = pair[mode]["page_gauge_fused_append_finalize"]["p50_us"] / 16
        out[mode] = {"fp16_append_us_per_step": round(a, 3), "fused_us_per_step": round(b, 3),
                     "incremental_us_per_step": round(max(0.0, b - a), 3)}
    return out


def _quantile(values, probability):
    """Linear-interpolation quantile (the reference summariser's,
    scripts/summarize_page_gauge_results.py:24-31)."""
    ordered = sorted(values)
    position = (len(ordered) - 1) * probability
    lower = int(position)
    upper = min(lower + 1, len(ordered) - 1)
    fraction = position - lower
    return ordered[lower] * (1.0 - fraction) + ordered[upper] * fraction


BOOTSTRAP_SEED = 20260815


def bootstrap_median_ci(values, samples: int = 20000, seed: int = BOOTSTRAP_SEED):
    """95 % bootstrap interval of the median over seeds (resampling with
    replacement; scripts/summarize_page_gauge_results.py:34-41)."""
    import random

    rng = random.Random(seed)
    medians = [statistics.median(rng.choices(values, k=len(values))) for _ in range(samples)]
    return [round(_quantile(medians, 0.025), 4), round(_quantile(medians, 0.975), 4)]


def seed_study(torch, decode, workloads, device, seeds, scrub, overhead, repeats: int = 20,
               frozen=None):
    """B1/49K over the validation seeds (scripts/run_page_gauge_validation.py:47-52):
    per seed, the paired INT8-vs-FP16 same-way protocol (cache-neutral after
    the reference's 256 MiB scrub, cache-hot), the attention-only speedup
    and the inclusive one (INT8 attention p50 + the fused-append increment
    per step, scripts/summarize_page_gauge_results.py:105-115); then the
    median over seeds and its 95 % bootstrap interval.  ``frozen``: a
    selection written by ``--pilot --freeze-splits``; each method then uses
    its frozen B1/49K split (0 = the planner), as the reference reuses its
    pilot's argmin for the validation seeds (:376-416)."""
    split = {"int8": 0, "fp16": 0}
    if frozen is not None:
        split = {m: int(frozen["shapes"]["b1_49k"][m]) for m in ("int8", "fp16")}
    per_seed = []
    for seed in seeds:
        w = workloads.b1_49k(seed, device=device, with_fp16_copy=True)
        out = torch.empty_like(w.query)
        lse = torch.empty(w.batch, 32, dtype=torch.float32, device=device)
        seg = decode.PageGaugeSegmentedDecode(torch.empty(64 << 20, dtype=torch.uint8, device=device))
        seg.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
                 w.tail_last_page_len, fixed_split_size=split["int8"] or None)
        int8 = seg.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                        w.value_center, out=out, lse=lse)
        f16 = decode.BatchDecodeWithPagedKVCacheWrapper(
            torch.empty(64 << 20, dtype=torch.uint8, device=device), "NHD")
        f16.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 32, 8, 128, 16,
                 kv_data_type=torch.float16, fixed_split_size=split["fp16"] or None)
        fp16 = f16.bind(w.query, (w.fp16_k, w.fp16_v), out=torch.empty_like(out),
                        lse=torch.empty_like(lse))
        pair = controlled_pair(torch, {"page_gauge_int8": int8, "fp16_same_way": fp16}, 3,
                               repeats, scrub)
        row = {"seed": seed}
        for mode in ("cache_neutral", "cache_hot"):
            a = pair[mode]["page_gauge_int8"]["p50_us"]
            b = pair[mode]["fp16_same_way"]["p50_us"]
            inc = overhead[mode]["incremental_us_per_step"]
            row[mode] = {"int8_p50_us": round(a, 3), "fp16_p50_us": round(b, 3),
                         "attention_only_speedup": round(b / a, 4),
                         "inclusive_speedup": round(b / (a + inc), 4)}
        per_seed.append(row)
        del w, seg, f16, int8, fp16
        torch.cuda.empty_cache()
    summary = {"seeds": list(seeds), "per_seed": per_seed,
               "append_increment_source": "append_overhead (B=1, paired, 16-step cycles)",
               "splits": {m: (v or "planner") for m, v in split.items()},
               "split_source": frozen.get("source") if frozen is not None else "the planner"}
    for mode in ("cache_neutral", "cache_hot"):
        # the reference resamples the inclusive ratios with the next seed
        # (scripts/summarize_page_gauge_results.py:56-69)
        for key, seed_offset in (("attention_only_speedup", 0), ("inclusive_speedup", 1)):
            values = [r[mode][key] for r in per_seed]
            summary.setdefault(mode, {})[key] = {
                "median": round(statistics.median(values), 4),
                "range": [min(values), max(values)],
                "seed_bootstrap_median_95_ci": (
                    bootstrap_median_ci(values, seed=BOOTSTRAP_SEED + seed_offset)
                    if len(values) > 1 else None)}
        summary[mode]["int8_p50_us_median"] = round(
            statistics.median(r[mode]["int8_p50_us"] for r in per_seed), 3)
    return summary


# (label, table entries, pages per item, KV heads per workgroup, groups in
# flight, lane pattern) of pg_probe_decode_walk.  3024 = 108 items of 28 pages
# (the planner's B1/49K items), 3040 = 95 x 32 = 190 x 16 = 380 x 8.
STREAM_PROBES = (
    ("decode pattern, 28-page items, 4 heads per workgroup, 2 groups in flight", 3024, 28, 4, 2, 0),
    ("decode pattern, 28-page items, 4 heads per workgroup, 1 group in flight", 3024, 28, 4, 1, 0),
    ("decode pattern, 16-page items, 8 heads per workgroup", 3040, 16, 8, 2, 0),
    ("decode pattern, 8-page items, 4 heads per workgroup", 3040, 8, 4, 2, 0),
    ("whole head rows, 32-page items, 4 heads per workgroup", 3040, 32, 4, 2, 1),
    ("whole head rows, 16-page items, 8 heads per workgroup", 3040, 16, 8, 2, 1),
    ("whole pages per workgroup, 16-page items", 3040, 16, 8, 2, 2),
    ("whole pages per workgroup, 8-page items", 3040, 8, 8, 2, 2),
)


STREAM_PROBES_16K = (
    ("decode pattern, 8-page items, 4 heads per workgroup", 1008, 8, 4, 2, 0),
    ("decode pattern, 12-page items, 4 heads per workgroup", 1008, 12, 4, 2, 0),
    ("decode pattern, 4-page items, 4 heads per workgroup", 1008, 4, 4, 1, 0),
    ("whole pages per workgroup, 8-page items", 1008, 8, 8, 2, 2),
    ("whole pages per workgroup, 4-page items", 1008, 4, 8, 1, 2),
)


STREAM_PROBES_B8 = (     # config 3, seed 20260840: its 8096 INT8 pages (the large plan)
    ("decode pattern, 32-page items, 8 heads per workgroup", 8096, 32, 8, 2, 0),
    ("decode pattern, 32-page items, 4 heads per workgroup", 8096, 32, 4, 2, 0),
    ("whole pages per workgroup, 16-page items", 8096, 16, 8, 2, 2),
)

STREAM_PROBES_4K = (
    ("decode pattern, 4-page items, 4 heads per workgroup, 1 group in flight", 240, 4, 4, 1, 0),
    ("decode pattern, 8-page items, 4 heads per workgroup", 240, 8, 4, 2, 0),
    ("whole pages per workgroup, 4-page items, 1 group in flight", 240, 4, 8, 1, 2),
)


def stream_probe(torch, w, bound, scrub, samples: int = 20, probes=STREAM_PROBES):
    """Load-only walks of the B1/49K INT8 pages (pg_probe_decode_walk) in the
    decode kernel's access pattern and in more favourable ones, cold (after
    the clean scrub) and hot, beside the decode's partial kernel timed the
    same way in the same process: how close the kernel comes to the stream of
    its own pattern.  Mean of dispatch-stamped durations."""
    lib = _probes()
    stream = torch.cuda.current_stream().cuda_stream
    sink = torch.empty(1 << 16, dtype=torch.int32, device=w.query.device)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(samples)]
    for pair in events:
        for e in pair:
            e.record()
    torch.cuda.synchronize()

    def timed(fn, before):
        for _ in range(2):
            if before is not None:
                before()
            fn(None, None)
        for a, b in events:
            if before is not None:
                before()
            fn(a.cuda_event, b.cuda_event)
        torch.cuda.synchronize()
        return 1e3 * statistics.fmean(a.elapsed_time(b) for a, b in events)

    rows = []
    for label, pages, per_item, heads, depth, mode in probes:
        def walk(start, stop, pages=pages, per_item=per_item, heads=heads, depth=depth, mode=mode):
            _probe_check(lib.pg_probe_decode_walk(
                w.k_codes.data_ptr(), w.v_codes.data_ptr(), w.old_indices.data_ptr(), pages,
                per_item, heads, depth, mode, sink.data_ptr(), sink.numel(), start, stop, stream))
        cold, hot = timed(walk, scrub), timed(walk, None)
        nbytes = pages * 2 * 16384
        rows.append({"probe": label, "pages": pages, "pages_per_item": per_item,
                     "heads_per_workgroup": heads, "groups_in_flight": depth, "mode": mode,
                     "workgroups": pages // per_item * (8 // heads),
                     "cold_us": round(cold, 2), "cold_gbps": round(nbytes / cold / 1e3, 1),
                     "hot_us": round(hot, 2), "hot_gbps": round(nbytes / hot / 1e3, 1)})
    kernel = {}
    for state, before in (("cold", scrub), ("hot", None)):
        for _ in range(3):
            if before is not None:
                before()
            bound()
        kernel[state] = round(1e3 * statistics.fmean(kernel_samples(torch, bound, samples, before)), 2)
    pages = int(w.old_indices.numel())
    best_cold = min(r["cold_us"] / r["pages"] for r in rows) * pages
    pattern_cold = rows[0]["cold_us"] / rows[0]["pages"] * pages
    tail_pages = int(w.tail_indices.numel())
    alg = w.algorithmic_bytes()
    kernel_gbps = alg / kernel["cold"] / 1e3
    return {"metric": "load-only stream of the INT8 pages vs the decode partial kernel",
            "unit": "us", "probes": rows,
            "decode_partial_kernel_us": kernel,
            "int8_pages": pages,
            "fp16_tail_pages": tail_pages,
            "kernel_over_own_pattern_cold": round(pattern_cold / kernel["cold"], 4),
            "kernel_over_best_probe_cold": round(best_cold / kernel["cold"], 4),
            # the kernel's algorithmic bytes (INT8 and FP16 pages, scales, query,
            # partials) per second against the probes' INT8 page rates
            "kernel_cold_gbps": round(kernel_gbps, 1),
            "kernel_gbps_over_own_pattern_cold": round(kernel_gbps / rows[0]["cold_gbps"], 4),
            "note": f"probe times scaled to the kernel's {pages} INT8 pages for the time ratios; "
                    f"the kernel also streams {tail_pages} FP16 tail pages "
                    f"({tail_pages * 65536 / 1e6:.1f} MB) and computes"}


# weight bytes of the config-5 decoder's projections (FP16 [rows, k])
DECODER_WEIGHTS = (("gate_up", 28672, 4096), ("down", 4096, 14336), ("qkv", 6144, 4096),
                   ("o", 4096, 4096), ("lm_head", 32768, 4096))


def weight_read_ceiling(torch, device, scrub, samples: int = 10):
    """Cold (after the clean scrub) nontemporal linear reads of each decoder
    projection's weight bytes (pg_probe_linear_read, best launch shape, mean
    of dispatch-stamped durations): the ceiling of the projection kernels,
    which read every weight byte once per step with the same loads."""
    lib = _probes()
    stream = torch.cuda.current_stream().cuda_stream
    sink = torch.empty(1 << 16, dtype=torch.int32, device=device)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(samples)]
    for pair in events:
        for e in pair:
            e.record()
    torch.cuda.synchronize()
    out = {}
    for name, rows, k in DECODER_WEIGHTS:
        nbytes = rows * k * 2
        buf = torch.ones(nbytes // 4, dtype=torch.int32, device=device)
        best = None
        for blocks in (512, 1024, 2048, 4096, 8192):
            for a, b in events:
                scrub()
                _probe_check(lib.pg_probe_linear_read(buf.data_ptr(), nbytes, sink.data_ptr(),
                                                      sink.numel(), blocks, a.cuda_event,
                                                      b.cuda_event, stream))
            torch.cuda.synchronize()
            t = 1e3 * statistics.fmean(a.elapsed_time(b) for a, b in events)
            best = t if best is None else min(best, t)
        out[name] = {"bytes": nbytes, "cold_read_us": round(best, 2),
                     "cold_read_gbps": round(nbytes / best / 1e3, 1)}
        del buf
    torch.cuda.empty_cache()
    return out


# Lanes of a trace row (pg_decode.hip, PG_TRACE builds): s_memrealtime marks
# at 100 MHz, then registers and notes.
TRACE_START, TRACE_IDS, TRACE_ISSUED, TRACE_SCALES = 0, 1, 2, 3
TRACE_K, TRACE_V, TRACE_DONE, TRACE_END = 4, 20, 36, 52
TRACE_XCC, TRACE_HWID, TRACE_ITEM, TRACE_KIND, TRACE_PAGES = 53, 54, 55, 56, 57
TRACE_TICK_US = 0.01
# combine kernel rows (written after the partial kernel's rows)
CTRACE_META, CTRACE_ROWS, CTRACE_MAX, CTRACE_SUMS, CTRACE_END = 1, 2, 3, 4, 5
CTRACE_KIND = 100


def _trace_stats(values):
    import numpy as np
    v = np.asarray(values, dtype=np.float64)
    if v.size == 0:
        return None
    q = np.percentile(v, [10, 50, 90])
    return {"p10": round(float(q[0]), 2), "p50": round(float(q[1]), 2),
            "p90": round(float(q[2]), 2), "max": round(float(v.max()), 2), "n": int(v.size)}


def trace_summary(rows_per_call, kernel_us, waves_per_block: int = 0):
    """Phase statistics (µs) of the per-wave trace rows of several calls.

    Times are relative to the first wave start on the same XCD in the same
    call: the s_memrealtime counters of different XCDs are not aligned (on
    this part XCDs 0 and 1 read about 1.9 µs behind the others, more than the
    kernel's own event duration allows as a real skew).  Per INT8
    wave: page-id round trip (ids - start), first group's data (K of group
    0 - its issue), and per group g: the wait for K (K[g] - done[g-1]), QK,
    softmax and the wait for V (V[g] - K[g]), PV issue (done[g] - V[g]).
    With ``waves_per_block``, also the p50 of each wave slot of a workgroup
    (KV head modulo the workgroup's waves): first issue after the page ids,
    first K data, end."""
    import numpy as np
    agg = {k: [] for k in ("start_at", "ids_rtt", "ids_at", "issued_at", "first_k_after_issue",
                           "first_k_at", "k_wait", "qk_to_v", "pv", "group_span", "end_at",
                           "end_at_fp16", "end_at_int8_last_group")}
    by_xcc, by_slot = {}, {}
    for rows in rows_per_call:
        r = rows.astype(np.int64) & 0xFFFFFFFF
        xcc = r[:, TRACE_XCC] & 0xF
        t0 = np.zeros(len(r), dtype=np.int64)
        for x in np.unique(xcc):
            t0[xcc == x] = r[xcc == x, TRACE_START].min()
        rel = lambda col: ((r[:, col] - t0) & 0xFFFFFFFF) * TRACE_TICK_US  # noqa: E731
        kind = r[:, TRACE_KIND]
        int8 = kind == 0
        agg["start_at"] += list(rel(TRACE_START))
        agg["ids_at"] += list(rel(TRACE_IDS))
        agg["ids_rtt"] += list(rel(TRACE_IDS) - rel(TRACE_START))
        agg["issued_at"] += list(rel(TRACE_ISSUED))
        agg["first_k_after_issue"] += list((rel(TRACE_K) - rel(TRACE_ISSUED))[int8])
        agg["first_k_at"] += list(rel(TRACE_K)[int8])
        agg["end_at"] += list(rel(TRACE_END))
        agg["end_at_fp16"] += list(rel(TRACE_END)[~int8])
        pages = r[:, TRACE_PAGES]
        groups = np.minimum((pages + 3) // 4, 16)
        for w in np.nonzero(int8)[0]:
            n = int(groups[w])
            k = [rel(TRACE_K + g)[w] for g in range(n)]
            v = [rel(TRACE_V + g)[w] for g in range(n)]
            d = [rel(TRACE_DONE + g)[w] for g in range(n)]
            for g in range(n):
                agg["qk_to_v"].append(v[g] - k[g])
                agg["pv"].append(d[g] - v[g])
                if g:
                    agg["k_wait"].append(k[g] - d[g - 1])
                    agg["group_span"].append(d[g] - d[g - 1])
            agg["end_at_int8_last_group"].append(d[n - 1])
        for x in np.unique(xcc):
            by_xcc.setdefault(int(x), []).extend(list(rel(TRACE_END)[xcc == x]))
        if waves_per_block:
            slot = (r[:, TRACE_ITEM] & 0xFF) % waves_per_block
            for w in range(waves_per_block):
                sel = int8 & (slot == w)
                d = by_slot.setdefault(w, {"issue_after_ids": [], "first_k_at": [], "end_at": []})
                d["issue_after_ids"] += list((rel(TRACE_ISSUED) - rel(TRACE_IDS))[sel])
                d["first_k_at"] += list(rel(TRACE_K)[sel])
                d["end_at"] += list(rel(TRACE_END)[sel])
    out = {k: _trace_stats(v) for k, v in agg.items()}
    if waves_per_block:
        out["p50_by_wave_slot"] = {w: {k: round(float(np.median(v)), 2) for k, v in d.items() if v}
                                   for w, d in sorted(by_slot.items())}
    out["end_at_p50_by_xcc"] = {x: round(float(np.median(v)), 2) for x, v in sorted(by_xcc.items())}
    out["kernel_event_mean_us"] = round(float(np.mean(kernel_us)), 3)
    out["waves_per_call"] = int(rows_per_call[0].shape[0])
    return out


def combine_trace_summary(partial_per_call, combine_per_call):
    """Phase statistics (µs) of the combine kernel's trace rows.

    Per XCD, times are relative to the first partial-kernel wave start on
    that XCD (the counters of one XCD agree with each other): the kernel
    boundary is the first combine wave start minus the last partial wave
    end, both on the same XCD.  Per combine wave: value center and item
    range arrival, partial rows arrival, the maximum over the rows, the sums
    (rows whose sums mark is unset are skipped), end."""
    import numpy as np
    agg = {k: [] for k in ("boundary", "start_spread", "meta_rtt", "rows_rtt", "max_after_rows",
                           "sums_after_max", "end_after_sums", "wave_life", "span")}
    for rp, rc in zip(partial_per_call, combine_per_call):
        p = rp.astype(np.int64) & 0xFFFFFFFF
        c = rc.astype(np.int64) & 0xFFFFFFFF
        if not np.all(c[:, TRACE_KIND] == CTRACE_KIND):
            raise RuntimeError("combine trace rows missing: is the buffer sized for both kernels?")
        pxcc, cxcc = p[:, TRACE_XCC] & 0xF, c[:, TRACE_XCC] & 0xF
        for x in np.unique(cxcc):
            pp, cc = p[pxcc == x], c[cxcc == x]
            if len(pp) == 0:
                continue
            t0 = pp[:, TRACE_START].min()
            rel = lambda rows, col: ((rows[:, col] - t0) & 0xFFFFFFFF) * TRACE_TICK_US  # noqa: E731
            start = rel(cc, TRACE_START)
            agg["boundary"].append(float(start.min() - rel(pp, TRACE_END).max()))
            agg["start_spread"] += list(start - start.min())
            agg["meta_rtt"] += list(rel(cc, CTRACE_META) - start)
            agg["rows_rtt"] += list(rel(cc, CTRACE_ROWS) - start)
            agg["max_after_rows"] += list(rel(cc, CTRACE_MAX) - rel(cc, CTRACE_ROWS))
            w0 = cc[:, CTRACE_SUMS] != 0
            agg["sums_after_max"] += list((rel(cc, CTRACE_SUMS) - rel(cc, CTRACE_MAX))[w0])
            agg["end_after_sums"] += list((rel(cc, CTRACE_END) - rel(cc, CTRACE_SUMS))[w0])
            agg["wave_life"] += list(rel(cc, CTRACE_END) - start)
            agg["span"].append(float(rel(cc, CTRACE_END).max() - start.min()))
    return {k: _trace_stats(v) for k, v in agg.items()}


def phase_trace(torch, decode, workloads, device, scrub, calls: int, dump: str = ""):
    """Per-wave phase trace of the partial kernel (trace build loaded), cold
    calls after the clean scrub, at B1/49K, 16K, 4K and config 3 (B8 ragged,
    first validation seed)."""
    from pagegauge_amd import _capi

    lib = _capi.library()
    if not hasattr(lib, "pg_trace_set_buffer"):
        raise RuntimeError("--trace needs a trace build (python -m pagegauge_amd.build --variant trace)")
    result, raw = {}, {}
    cases = (("b1_49k", lambda: workloads.b1_49k(workloads.VALIDATION_SEEDS[0], device=device)),
             ("b1_16k", lambda: workloads.build_decode_workload([16384 + 16], workloads.VALIDATION_SEEDS[0],
                                                                device=device)),
             ("config1_4k", lambda: workloads.single_4k(workloads.VALIDATION_SEEDS[0], device=device)),
             ("config3_b8_ragged", lambda: workloads.build_decode_workload(
                 workloads.ragged_lengths(workloads.VALIDATION_SEEDS[0]), workloads.VALIDATION_SEEDS[0],
                 device=device)))
    for name, make in cases:
        w = make()
        dec = decode.PageGaugeSegmentedDecode(torch.empty(64 << 20, dtype=torch.uint8, device=device))
        dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
                 w.tail_last_page_len)
        bound = dec.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                         w.value_center, out=torch.empty_like(w.query),
                         lse=torch.empty(w.batch, 32, dtype=torch.float32, device=device))
        waves = dec.num_work_items * 8
        combine_waves = w.batch * 32 * 4 * 4      # (request, query head) x 4 quarters x 4 waves
        buf = torch.zeros((waves + combine_waves) * 64, dtype=torch.int32, device=device)
        _capi.check(lib.pg_trace_set_buffer(buf.data_ptr(), buf.numel() * 4), "trace")
        for _ in range(3):
            scrub()
            bound()
        rows, combine_rows, kernel = [], [], []
        for _ in range(calls):
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            stop.record()
            buf.zero_()
            scrub()
            bound.partial_timed(start.cuda_event, stop.cuda_event)
            bound.combine()
            torch.cuda.synchronize()
            kernel.append(1e3 * start.elapsed_time(stop))
            host = buf.view(waves + combine_waves, 64).cpu().numpy()
            rows.append(host[:waves].copy())
            combine_rows.append(host[waves:].copy())
        _capi.check(lib.pg_trace_set_buffer(None, 0), "trace")
        if dump:
            import numpy as np
            raw[f"{name}_partial"] = np.stack(rows)
            raw[f"{name}_combine"] = np.stack(combine_rows)
            raw[f"{name}_kernel_us"] = np.asarray(kernel)
        result[name] = {"work_items": dec.num_work_items,
                        "waves_per_block": int(dec._state.plan.waves_per_block),
                        **trace_summary(rows, kernel, int(dec._state.plan.waves_per_block)),
                        "combine": combine_trace_summary(rows, combine_rows)}
        del w, dec, bound, buf
        torch.cuda.empty_cache()
    if dump:
        import numpy as np
        np.savez_compressed(dump, **raw)
    return result


PILOT_SPLITS = (0, 8, 16, 28, 48, 64)


def frozen_selection(pilot: dict) -> dict:
    """The reference's FROZEN_SELECTION.json of a pilot sweep
    (scripts/run_page_gauge_validation.py:295-316, :398-418): per shape and
    method the argmin split of the cold call p50 (0 = the planner)."""
    shapes = {}
    for name, row in pilot.items():
        if isinstance(row, dict) and "int8" in row:
            shapes[name] = {m: int(row[m]["argmin"]) for m in ("int8", "fp16")}
            shapes[name]["rows"] = {m: {k: v["call_p50_us"] for k, v in row[m].items()
                                        if isinstance(v, dict)} for m in ("int8", "fp16")}
    return {"source": f"pilot sweep, seed {PILOT_SEED_NOTE}, cold (clean 1 GiB read scrub)",
            "selection_timing_mode": "cache_neutral", "shapes": shapes}


PILOT_SEED_NOTE = "20260814 (B1 shapes) / the validation seeds (B8 ragged)"


def pilot_sweep(torch, decode, workloads, device, scrub, samples: int = 30):
    """The reference's pilot sweep (scripts/run_page_gauge_validation.py:277-297,
    :376-416): for each method (INT8 PageGauge, FP16 same-way) every split
    in PILOT_SPLITS (0 = this build's planner; otherwise FlashInfer's
    fixed_split_size: pages per work item) is timed cold (p50 of the whole
    call after the read-only 1 GiB scrub), the argmin is frozen per method,
    and the planner's pick is compared with it.  Shapes: B1/49K (pilot seed
    20260814), B8 ragged (3 validation seeds), B1 at 16K and at 64K."""
    shapes = [("b1_49k", [49152], workloads.PILOT_SEED)]
    shapes += [(f"b8_ragged_{s}", workloads.ragged_lengths(s), s)
               for s in workloads.VALIDATION_SEEDS[:3]]
    shapes += [("b1_16k", [16384], workloads.PILOT_SEED), ("b1_64k", [65536], workloads.PILOT_SEED)]
    result = {"splits": list(PILOT_SPLITS), "state": "cold (1 GiB read scrub), p50 of the call"}
    for name, lengths, seed in shapes:
        w = workloads.build_decode_workload(lengths, seed, device=device, with_fp16_copy=True)
        out = torch.empty_like(w.query)
        lse = torch.empty(w.batch, 32, dtype=torch.float32, device=device)
        ws = torch.empty(64 << 20, dtype=torch.uint8, device=device)
        row = {}
        for method in ("int8", "fp16"):
            times = {}
            for split in PILOT_SPLITS:
                if method == "int8":
                    d = decode.PageGaugeSegmentedDecode(ws)
                    d.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr,
                           w.tail_indices, w.tail_last_page_len, fixed_split_size=split or None)
                    b = d.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                               (w.tail_k, w.tail_v), w.value_center, out=out, lse=lse)
                else:
                    d = decode.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
                    d.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 32, 8, 128, 16,
                           kv_data_type=torch.float16, fixed_split_size=split or None)
                    b = d.bind(w.query, (w.fp16_k, w.fp16_v), out=out, lse=lse)
                for _ in range(3):
                    scrub()
                    b()
                ms = call_samples(torch, b, samples, scrub)
                times[str(split)] = {"call_p50_us": round(1e3 * statistics.median(ms), 2),
                                     "items": d.num_work_items}
            best = min(times, key=lambda k: times[k]["call_p50_us"])
            times["argmin"] = best
            times["planner_over_argmin"] = round(times["0"]["call_p50_us"] /
                                                 times[best]["call_p50_us"], 4)
            row[method] = times
        result[name] = {"lengths": lengths if len(lengths) <= 8 else len(lengths), **row}
        print(json.dumps({name: result[name]}), file=sys.stderr, flush=True)
        del w
        torch.cuda.empty_cache()
    return result


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path is a single-GPU decode, and this run "
              f"uses one GPU); --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    if args.trace:
        args.library_variant = args.trace
    if args.library_variant:
        from pagegauge_amd import _capi, build
        if not build.variant_is_current(args.library_variant):
            print(f"the {args.library_variant} build is missing or older than the sources: run "
                  f"python -m pagegauge_amd.build --variant {args.library_variant}", file=sys.stderr)
            return 2
        _capi.LIBRARY_PATH = build.variant_library(args.library_variant)
    from pagegauge_amd import decode, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.decoder_only:
        print(json.dumps(decoder_config5(torch, device, args.decoder_repeats)), flush=True)
        return 0
    if args.trace:
        buf = torch.ones((args.big_scrub_mib << 20) // 4, dtype=torch.int32, device=device)
        sink = torch.empty((), dtype=torch.int32, device=device)
        print(json.dumps({"trace_build": args.trace, **phase_trace(
            torch, decode, workloads, device, lambda: torch.amax(buf, dim=0, out=sink),
            args.trace_calls, args.trace_dump)}), flush=True)
        return 0
    if args.paper_only:
        buf = torch.ones((args.big_scrub_mib << 20) // 4, dtype=torch.int32, device=device)
        sink = torch.empty((), dtype=torch.int32, device=device)
        print(json.dumps(paper_b4_20k(torch, decode, workloads, device,
                                      lambda: torch.amax(buf, dim=0, out=sink), 60)), flush=True)
        return 0
    t_setup = time.perf_counter()
    if args.pmc_calls and args.workload == "config1":
        w = workloads.single_4k(args.seed, device=device, with_fp16_copy=not args.no_fp16)
    elif args.pmc_calls and args.workload == "b1_16k":
        w = workloads.build_decode_workload([16384 + 16], args.seed, device=device,
                                            with_fp16_copy=not args.no_fp16)
    elif args.pmc_calls and args.workload == "serving_b256":
        w = workloads.serving_b256(device=device, with_fp16_copy=not args.no_fp16)
    else:
        w = workloads.b1_49k(args.seed, device=device, with_fp16_copy=not args.no_fp16)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    workspace = torch.empty(64 << 20, dtype=torch.uint8, device=device)
    out = torch.empty_like(w.query)
    lse = torch.empty(w.batch, 32, dtype=torch.float32, device=device)
    dec = decode.PageGaugeSegmentedDecode(workspace)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len, fixed_split_size=args.split or None)
    bound = dec.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                     w.value_center, out=out, lse=lse)

    # rmw scrub: the reference protocol (scripts/benchmark_flashinfer_page_affine_int8.py:651-655)
    scrub_rmw_buf = torch.zeros(args.scrub_mib * (1 << 20) // 4, dtype=torch.int32, device=device)
    scrub_rmw = lambda: scrub_rmw_buf.add_(1)  # noqa: E731
    # clean scrub: read 1 GiB (> the 256 MB MALL) and write one word
    scrub_clean_buf = torch.ones(args.big_scrub_mib * (1 << 20) // 4, dtype=torch.int32, device=device)
    scrub_sink = torch.empty((), dtype=torch.int32, device=device)
    scrub_clean = lambda: torch.amax(scrub_clean_buf, dim=0, out=scrub_sink)  # noqa: E731

    if args.pmc_calls:
        driven, what = bound, "int8"
        if args.pmc_fp16:
            if w.fp16_k is None:
                raise SystemExit("--pmc-fp16 needs the FP16 copy (drop --no-fp16)")
            wrap16 = decode.BatchDecodeWithPagedKVCacheWrapper(
                torch.empty(64 << 20, dtype=torch.uint8, device=device), "NHD")
            wrap16.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 32, 8, 128, 16,
                        kv_data_type=torch.float16)
            driven = wrap16.bind(w.query, (w.fp16_k, w.fp16_v), out=torch.empty_like(w.query),
                                 lse=torch.empty_like(lse))
            what = "fp16_same_way"
        print(json.dumps({**pmc_driver(torch, driven, args.pmc_calls, scrub_clean, device),
                          "call": what, "workload": args.workload,
                          "library_variant": args.library_variant}), flush=True)
        return 0
    if args.pilot:
        pilot = pilot_sweep(torch, decode, workloads, device, scrub_clean)
        if args.freeze_splits:
            Path(args.freeze_splits).write_text(json.dumps(frozen_selection(pilot), indent=1) + "\n")
        print(json.dumps(pilot), flush=True)
        return 0
    if args.stream_probe:
        result = {"b1_49k": stream_probe(torch, w, bound, scrub_clean)}
        # the config-5 decoder's per-layer shape: 16K context (1008 INT8 pages + the ring)
        w16 = workloads.build_decode_workload([16384 + 16], args.seed, device=device)
        d16 = decode.PageGaugeSegmentedDecode(torch.empty(64 << 20, dtype=torch.uint8, device=device))
        d16.plan(w16.old_indptr, w16.old_indices, w16.old_last_page_len, w16.tail_indptr,
                 w16.tail_indices, w16.tail_last_page_len)
        b16 = d16.bind(w16.query, (w16.k_codes, w16.v_codes), w16.k_scale, w16.v_scale,
                       (w16.tail_k, w16.tail_v), w16.value_center, out=torch.empty_like(w16.query),
                       lse=torch.empty(1, 32, dtype=torch.float32, device=device))
        result["b1_16k"] = stream_probe(torch, w16, b16, scrub_clean, probes=STREAM_PROBES_16K)
        del w16, d16, b16
        # config 1: 4096 tokens (240 INT8 pages + the ring)
        w4 = workloads.single_4k(args.seed, device=device)
        d4 = decode.PageGaugeSegmentedDecode(torch.empty(64 << 20, dtype=torch.uint8, device=device))
        d4.plan(w4.old_indptr, w4.old_indices, w4.old_last_page_len, w4.tail_indptr,
                w4.tail_indices, w4.tail_last_page_len)
        b4 = d4.bind(w4.query, (w4.k_codes, w4.v_codes), w4.k_scale, w4.v_scale,
                     (w4.tail_k, w4.tail_v), w4.value_center, out=torch.empty_like(w4.query),
                     lse=torch.empty(1, 32, dtype=torch.float32, device=device))
        result["config1_4k"] = stream_probe(torch, w4, b4, scrub_clean, probes=STREAM_PROBES_4K)
        del w4, d4, b4
        # config 3 (first seed), the large plan
        w8 = workloads.b8_ragged(workloads.VALIDATION_SEEDS[0], device=device)
        d8 = decode.PageGaugeSegmentedDecode(torch.empty(64 << 20, dtype=torch.uint8, device=device))
        d8.plan(w8.old_indptr, w8.old_indices, w8.old_last_page_len, w8.tail_indptr,
                w8.tail_indices, w8.tail_last_page_len)
        b8 = d8.bind(w8.query, (w8.k_codes, w8.v_codes), w8.k_scale, w8.v_scale,
                     (w8.tail_k, w8.tail_v), w8.value_center, out=torch.empty_like(w8.query),
                     lse=torch.empty(8, 32, dtype=torch.float32, device=device))
        result["config3_b8_ragged"] = stream_probe(torch, w8, b8, scrub_clean, probes=STREAM_PROBES_B8)
        del w8, d8, b8
        # the serving-sized batch of the bench line (256 requests, the large plan)
        wb = workloads.serving_b256(device=device)
        db = decode.PageGaugeSegmentedDecode(torch.empty(128 << 20, dtype=torch.uint8, device=device))
        db.plan(wb.old_indptr, wb.old_indices, wb.old_last_page_len, wb.tail_indptr,
                wb.tail_indices, wb.tail_last_page_len)
        bb = db.bind(wb.query, (wb.k_codes, wb.v_codes), wb.k_scale, wb.v_scale,
                     (wb.tail_k, wb.tail_v), wb.value_center, out=torch.empty_like(wb.query),
                     lse=torch.empty(256, 32, dtype=torch.float32, device=device))
        n_int8 = int(wb.old_indptr[-1]) // 64 * 64     # whole items of every probe
        result["serving_b256"] = stream_probe(torch, wb, bb, scrub_clean, probes=(
            ("decode pattern, 32-page items, 8 heads per workgroup", n_int8, 32, 8, 2, 0),
            ("decode pattern, 64-page items, 8 heads per workgroup", n_int8, 64, 8, 2, 0),
            ("whole pages per workgroup, 16-page items", n_int8, 16, 8, 2, 2)))
        del wb, db, bb
        result["decoder_weight_reads"] = weight_read_ceiling(torch, device, scrub_clean)
        print(json.dumps(result), flush=True)
        return 0

    # contract timed region: K cold steps bracketed by synchronize
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    int8 = measure(torch, bound, args, scrub_clean, scrub_rmw)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - wall0
    # the same call captured in a HIP graph (as the decoder's step graphs run it)
    graph_ms = graph_call_samples(
        torch, lambda s: dec.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                                  (w.tail_k, w.tail_v), w.value_center, out=out, lse=lse,
                                  stream=s), args.steps, scrub_clean)
    int8["cold_clean_1gib_graph"] = {"call": summarize(graph_ms),
                                     "fixed_cost": graph_fixed_cost(torch, scrub_clean)}
    bound()
    torch.cuda.synchronize()
    gpu_out = out.detach().cpu().numpy()
    gpu_lse = lse.detach().cpu().numpy()

    alg_bytes = w.algorithmic_bytes()
    kernel_mean_us = int8["cold_clean_1gib"]["kernel"]["mean_us"]
    call_p50_us = int8["cold_clean_1gib"]["call"]["p50_us"]
    achieved = alg_bytes / (kernel_mean_us * 1e-6) / 1e9

    fp16 = None
    if not args.no_fp16:
        ws16 = torch.empty(64 << 20, dtype=torch.uint8, device=device)
        out16 = torch.empty_like(w.query)
        lse16 = torch.empty_like(lse)
        wrap16 = decode.BatchDecodeWithPagedKVCacheWrapper(ws16, "NHD")
        wrap16.plan(w.fp16_indptr, w.fp16_indices, w.fp16_last_page_len, 32, 8, 128, 16,
                    kv_data_type=torch.float16, fixed_split_size=None)
        bound16 = wrap16.bind(w.query, (w.fp16_k, w.fp16_v), out=out16, lse=lse16)
        fp16 = measure(torch, bound16, args, scrub_clean, scrub_rmw)
        fp16_bytes = w.fp16_algorithmic_bytes()
        fp16["algorithmic_bytes"] = fp16_bytes
        fp16["split_pages"] = wrap16.split_pages
        fp16["achieved_gbps_cold_kernel"] = fp16_bytes / (fp16["cold_clean_1gib"]["kernel"]["mean_us"] * 1e-6) / 1e9
        # the reference's A/B, B/A paired protocol on the same two calls
        fp16["paired_with_int8"] = controlled_pair(
            torch, {"page_gauge_int8": bound, "fp16_same_way": bound16}, 3,
            max(20, args.steps // 2), scrub_rmw)

    sweep = {}
    for item in [s for s in args.sweep.split(",") if s.strip()]:
        split = int(item)
        d2 = decode.PageGaugeSegmentedDecode(workspace)
        d2.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
                w.tail_last_page_len, fixed_split_size=split)
        b2 = d2.bind(w.query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                     w.value_center, out=out, lse=lse)
        k_ms, c_ms = timed_calls(torch, b2, max(20, args.steps // 2), scrub=scrub_clean)
        sweep[str(split)] = {"items": d2.num_work_items, "kernel_p50_us": 1e3 * statistics.median(k_ms),
                             "call_p50_us": 1e3 * statistics.median(c_ms)}

    other = None
    if not args.no_configs:
        other = {"config1_b1_4k": decode_config(
            torch, decode, workloads.single_4k(args.seed, device=device, with_fp16_copy=True),
            scrub_clean, 30)}
        # config 5's per-layer decode shape: 16K context (1008 INT8 pages + the ring)
        other["b1_16k"] = decode_config(
            torch, decode, workloads.build_decode_workload([16384 + 16], args.seed, device=device,
                                                           with_fp16_copy=True), scrub_clean, 30)
        torch.cuda.empty_cache()
        # B1/49K through the heterogeneous one-table decode (same pages)
        out_h = torch.empty_like(w.query)
        het = heterogeneous_call(torch, decode, w, device, out_h)
        for _ in range(3):
            scrub_clean()
            het()
        het_ms = call_samples(torch, het, 40, scrub_clean)
        torch.cuda.synchronize()
        other["b1_49k_heterogeneous"] = {
            "call_p50_us": round(1e3 * statistics.median(het_ms), 3),
            "segmented_call_p50_us": round(call_p50_us, 3),
            "max_abs_vs_segmented": float(np.abs(out_h.cpu().numpy().astype(np.float32)
                                                 - gpu_out.astype(np.float32)).max())}
        del het, out_h
        # B1/49K with the reference driver's own page table: physical pages in
        # logical order (scripts/benchmark_flashinfer_page_affine_int8.py:463)
        wi = workloads.b1_49k(args.seed, device=device, shuffle_pages=False)
        other["b1_49k_identity_page_table"] = decode_config(torch, decode, wi, scrub_clean, 40)
        del wi
        ragged = {}
        for seed in workloads.VALIDATION_SEEDS[:3]:
            wr = workloads.b8_ragged(seed, device=device, with_fp16_copy=True)
            ragged[str(seed)] = decode_config(torch, decode, wr, scrub_clean, 30)
            del wr
            torch.cuda.empty_cache()
        other["config3_b8_ragged"] = ragged
        # a serving-sized batch: 256 requests of 16-240 INT8 pages (U, seeded)
        # behind full 16-page rings, in one shuffled pool
        wb = workloads.serving_b256(device=device, with_fp16_copy=True)
        other["serving_b256"] = decode_config(torch, decode, wb, scrub_clean, 20)
        other["serving_b256"]["total_tokens"] = sum(wb.lengths)
        del wb
        torch.cuda.empty_cache()
        other["config4_update"] = update_config4(torch, device, 50)
        other["exact_tail_merge_center"] = exact_tail_merge_line(torch, device, scrub_clean)
        other["paper_b4_20k"] = paper_b4_20k(torch, decode, workloads, device, scrub_clean, 60)
    if not args.no_decoder:
        other = other or {}
        other["config5_decoder"] = decoder_config5(torch, device, args.decoder_repeats)
        other["paper_b4_20k_decoder"] = decoder_b4_20k(torch, device, 2)

    peak = measure_peak(torch, device, w, scrub_clean)
    overhead = append_overhead(torch, device, scrub_rmw)
    seeds = None
    if args.seeds > 0 and not args.no_fp16:
        frozen = json.loads(Path(args.frozen_splits).read_text()) if args.frozen_splits else None
        seeds = seed_study(torch, decode, workloads, device,
                           workloads.VALIDATION_SEEDS[:args.seeds], scrub_rmw, overhead,
                           frozen=frozen)

    cpu = None
    parity = None
    if not args.no_cpu:
        base = cpu_baseline(torch, w, device, configs=not args.no_configs)
        b1 = base.pop("b1_49k")
        ref_out, ref_lse = b1.pop("out").numpy(), b1.pop("lse").numpy()
        host = base.pop("host")
        cpu = {
            "value": round(b1["ms"]["p50_us"], 1),
            "unit": "us/call",
            "cores": host["torch_threads"],
            "kind": "port",
            "sample": (f"the bench workload itself: full B1/49K decode of the same inputs (3056 INT8 "
                       f"+ 16 FP16 pages dequantised, dense float32 softmax, value center), torch "
                       f"CPU restatement (oracle/cpu_baseline.py) on {host['torch_threads']} threads, "
                       f"3 warm-ups + {b1['ms']['samples']} timed calls"),
            "p05_us": round(b1["ms"]["p05_us"], 1), "p95_us": round(b1["ms"]["p95_us"], 1),
            "cpu_model": host["cpu_model"], "cpu_count": host["cpu_count"],
            "other_configs": base,
        }
        parity = {
            "oracle": "torch-CPU float32 dense decode (oracle/cpu_baseline.py)",
            "max_abs_out": float(np.abs(gpu_out.astype(np.float64) - ref_out.astype(np.float64)).max()),
            "max_abs_lse": float(np.abs(gpu_lse.astype(np.float64) - ref_lse.astype(np.float64)).max()),
            "tolerance_out": 2e-3,
        }

    result = {
        "metric": "B1/49K INT8 paged-decode us/call (HBM-cold after a clean 1 GiB read scrub; whole call incl. combine)",
        "value": round(call_p50_us, 3),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(call_p50_us / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 codes (int32 MFMA accumulate) + fp16 tail, fp32 softmax",
        "data": "synthetic (seeded N(0,1) K/V, x8 outliers on 4/128 channels, permuted page table)",
        "config": {
            "workload": "b1_49k: B=1, 49152 tokens = 3056 INT8 pages + 16 FP16 tail pages, "
                        "Hq=32 Hkv=8 D=128 page 16",
            "seed": args.seed,
            "split_pages": dec.split_pages,
            "tail_split_pages": dec.tail_split_pages,
            "work_items": dec.num_work_items,
            "step": "one decode call (pg_decode_run) after an untimed read-only 1 GiB scrub",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_partial_kernel",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "peak_source": "MI355X HBM3E specification",
            "peak_measured": peak,
            "frac_of_measured_read_1gib": round(achieved / peak["read_1gib_gbps"], 4),
            "frac_of_measured_cold_101mb_read": round(achieved / peak["cold_read_101mb_gbps"], 4),
            "frac_of_measured_cold_page_walk": round(achieved / peak["cold_page_walk_b1_49k_gbps"], 4),
            "traffic": committed_traffic(ROOT),
            "traffic_source": "profiles/decode_partial_b1_49k_pmc.md (FETCH_SIZE + WRITE_SIZE, "
                              "calibrated by a plain copy)",
            "algorithmic_bytes": alg_bytes,
            "kernel_mean_us": round(kernel_mean_us, 3),
        },
        "cpu_baseline": cpu,
        "timings_int8": {k: v for k, v in int8.items() if not k.startswith("_")},
        "timings_fp16_same_way": None if fp16 is None else {k: v for k, v in fp16.items() if not k.startswith("_")},
        "speedup_vs_fp16_same_way": None if fp16 is None else {
            mode: round(fp16[mode]["call"]["p50_us"] / int8[mode]["call"]["p50_us"], 4)
            for mode in ("cold_clean_1gib", "cold_rmw_256mib", "hot") if mode in int8},
        "fused_append_increment_b1": overhead,
        "validation_seeds_b1_49k": seeds,
        "parity_vs_oracle": parity,
        "library_variant": args.library_variant,
        "library_flags": {src: flags for src, flags in build_sources().items() if flags},
        "output_sha256": hashlib.sha256(gpu_out.tobytes() + gpu_lse.tobytes()).hexdigest(),
        "split_sweep": sweep or None,
        "other_configs": other,
        "wall_s_timed_region": round(wall_s, 3),
        "setup_s": round(setup_s, 2),
        "device": torch.cuda.get_device_name(device),
        "host_cpus": os.cpu_count(),
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
