"""GPU: the update and decode entry points inside a captured HIP graph.

The reference keeps both ABIs graph-capturable (caller-owned buffers, no
allocation, no host sync; scripts/benchmark_page_gauge_transformer.py
:2817-3228 replays a captured decoder step with a device position).  Each
replay is checked against the eager result, with eager work and
synchronisations between replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pg_oracle as oracle
from tests.helpers import cpu

pytestmark = pytest.mark.gpu


def _rand(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.float16)


def test_config4_update_steps_replay_in_a_graph(cuda):
    from pagegauge_amd import runtime

    ext = runtime.load_append_extension()
    gen = torch.Generator().manual_seed(20260840)
    start = [4096, 4099, 8192, 8199, 12288, 12299, 16384, 16398]
    batch, ring_pages, steps = 8, 16, 16
    code_pages = (max(start) + steps + 15) // 16
    cos_np, sin_np = oracle.rope_tables(max(start) + steps)
    cos, sin = torch.from_numpy(cos_np).to(cuda), torch.from_numpy(sin_np).to(cuda)
    kc = _rand(gen, batch, 8, 128, scale=0.1).to(cuda)
    vc = _rand(gen, batch, 8, 128, scale=0.1).to(cuda)
    q = [_rand(gen, batch, 32, 128).to(cuda) for _ in range(steps)]
    k = [_rand(gen, batch, 8, 128).to(cuda) for _ in range(steps)]
    v = [_rand(gen, batch, 8, 128).to(cuda) for _ in range(steps)]
    pos = [torch.tensor([s + t for s in start], dtype=torch.int32, device=cuda) for t in range(steps)]
    ring0 = _rand(gen, batch * ring_pages, 16, 8, 128).to(cuda)

    def fresh():
        return [ring0.clone(), ring0.clone(),
                torch.zeros(batch * code_pages, 16, 8, 128, dtype=torch.int8, device=cuda),
                torch.zeros(batch * code_pages, 16, 8, 128, dtype=torch.int8, device=cuda),
                torch.zeros(batch * code_pages, 8, dtype=torch.float16, device=cuda),
                torch.zeros(batch * code_pages, 8, dtype=torch.float16, device=cuda)]

    def run_steps(state, rq):
        for t in range(steps):
            ext.rope_append_page_gauge_positions(q[t], k[t], v[t], cos, sin, pos[t], kc, vc, rq,
                                                 *state, 0)

    eager = fresh()
    eager_rq = torch.zeros(batch, 32, 128, dtype=torch.float16, device=cuda)
    run_steps(eager, eager_rq)
    torch.cuda.synchronize()
    want = [cpu(t).copy() for t in eager] + [cpu(eager_rq).copy()]

    graph_state = fresh()
    graph_rq = torch.zeros(batch, 32, 128, dtype=torch.float16, device=cuda)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run_steps(graph_state, graph_rq)
    torch.cuda.synchronize()
    for replay in range(3):
        print("graph replay", replay, flush=True)
        for dst, src in zip(graph_state, fresh()):      # eager work between replays
            dst.copy_(src)
        graph_rq.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [cpu(t) for t in graph_state] + [cpu(graph_rq)]
        for g, w in zip(got, want):
            assert np.array_equal(np.ascontiguousarray(g).view(np.uint8),
                                  np.ascontiguousarray(w).view(np.uint8)), replay


def test_bound_decode_replays_in_a_graph(cuda):
    from pagegauge_amd import decode, workloads

    w = workloads.build_decode_workload([8192, 2048], seed=20260841, device=cuda)
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=cuda)
    dec = decode.PageGaugeSegmentedDecode(ws)
    dec.plan(w.old_indptr, w.old_indices, w.old_last_page_len, w.tail_indptr, w.tail_indices,
             w.tail_last_page_len)
    out = torch.empty_like(w.query)
    lse = torch.empty(w.batch, 32, dtype=torch.float32, device=cuda)
    query = w.query.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        bound = dec.bind(query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale,
                         (w.tail_k, w.tail_v), w.value_center, out=out, lse=lse)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        bound()
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(3)
    for replay in range(3):
        print("decode graph replay", replay, flush=True)
        new_q = _rand(gen, *query.shape).to(cuda)
        query.copy_(new_q)                       # the graph reads the query buffer in place
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got_out, got_lse = cpu(out).copy(), cpu(lse).copy()
        eager_out = torch.empty_like(out)
        eager_lse = torch.empty_like(lse)
        dec.run(query, (w.k_codes, w.v_codes), w.k_scale, w.v_scale, (w.tail_k, w.tail_v),
                w.value_center, out=eager_out, lse=eager_lse)
        torch.cuda.synchronize()
        assert np.array_equal(got_out.view(np.uint16), cpu(eager_out).view(np.uint16)), replay
        assert np.array_equal(got_lse.view(np.uint32), cpu(eager_lse).view(np.uint32)), replay
