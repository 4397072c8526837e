"""The HBM read probes (libpagegauge_bench.so, bench.py's roofline peak):
they launch, leave the sink untouched for data that cannot hit the sink's
condition, time themselves through dispatch-stamped events, and reject bad
arguments."""

from __future__ import annotations

import pytest
import torch

from pagegauge_amd import _capi

pytestmark = pytest.mark.gpu


def test_probes_read_and_time_themselves(cuda):
    lib = _capi.bench_library()
    stream = torch.cuda.current_stream().cuda_stream
    data = torch.zeros(1 << 20, dtype=torch.int32, device=cuda)
    sink = torch.full((4096,), 7, dtype=torch.int32, device=cuda)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    stop.record()
    torch.cuda.synchronize()
    assert lib.pg_probe_linear_read(data.data_ptr(), data.numel() * 4, sink.data_ptr(),
                                    sink.numel(), 512, start.cuda_event, stop.cuda_event,
                                    stream) == 0
    pages = torch.zeros(8, 16, 8, 128, dtype=torch.int8, device=cuda)
    ids = torch.tensor([5, 0, 7, 2], dtype=torch.int32, device=cuda)
    assert lib.pg_probe_page_walk(pages.data_ptr(), pages.data_ptr(), ids.data_ptr(), 4, 2, 16384,
                                  sink.data_ptr(), sink.numel(), None, None, stream) == 0
    torch.cuda.synchronize()
    assert start.elapsed_time(stop) > 0.0
    assert bool((sink == 7).all())             # zero data never meets the write condition
    assert lib.pg_probe_linear_read(data.data_ptr(), 17, sink.data_ptr(), sink.numel(), 1, None,
                                    None, stream) == 1
    assert "16-byte" in lib.pg_last_error().decode()
    assert lib.pg_probe_page_walk(None, None, None, 1, 1, 16, sink.data_ptr(), sink.numel(), None,
                                  None, stream) == 1


def test_decode_walk_probe_reads_in_every_mode(cuda):
    lib = _capi.bench_library()
    stream = torch.cuda.current_stream().cuda_stream
    pages = torch.zeros(16, 16, 8, 128, dtype=torch.int8, device=cuda)
    ids = torch.randperm(16, dtype=torch.int32).to(cuda)
    sink = torch.full((64,), 7, dtype=torch.int32, device=cuda)
    for per_item, heads, depth, mode in ((4, 4, 1, 0), (8, 4, 2, 0), (16, 8, 2, 0), (8, 4, 2, 1),
                                         (8, 8, 1, 2)):
        assert lib.pg_probe_decode_walk(pages.data_ptr(), pages.data_ptr(), ids.data_ptr(), 16,
                                        per_item, heads, depth, mode, sink.data_ptr(),
                                        sink.numel(), None, None, stream) == 0, lib.pg_last_error()
    torch.cuda.synchronize()
    assert bool((sink == 7).all())
