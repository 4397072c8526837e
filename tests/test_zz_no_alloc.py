"""The no-allocation center reduction (pg_token_major_centers_noalloc).

It must give bit-identical centers to pg_token_major_centers (the entry point
with a caller workspace, itself pinned against the exact-rational oracle in
tests/test_gpu_prefill.py), called through the C ABI, on consecutive calls
of decreasing size: the device scratch array keeps the previous call's chunk
sums, so a second, smaller call that read any stale sum would differ.
"""

from __future__ import annotations

import pytest
import torch

from pagegauge_amd import _capi

pytestmark = pytest.mark.gpu


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _inputs(tokens: int, heads: int, seed: int, device, stride_pad: int = 0):
    """Token-major K and V views [tokens, heads, 128] with row stride
    heads*128 + stride_pad (a K/V slice of a fused projection when padded)."""
    gen = torch.Generator().manual_seed(seed)
    row = heads * 128 + stride_pad
    k = (torch.randn(tokens, row, generator=gen) * 3).half().to(device)
    v = (torch.randn(tokens, row, generator=gen) * 0.5).half().to(device)
    view = lambda t: t[:, :heads * 128].view(tokens, heads, 128) if stride_pad else t.view(tokens, heads, 128)  # noqa: E731
    return view(k), view(v), row


def _with_workspace(k, v, row, tokens, heads):
    lib = _capi.library()
    need = int(lib.pg_token_major_centers_workspace_bytes(tokens, heads))
    ws = torch.empty(need, dtype=torch.uint8, device=k.device)
    kc = torch.empty(heads, 128, dtype=torch.float16, device=k.device)
    vc = torch.empty_like(kc)
    _capi.call("pg_token_major_centers", k.data_ptr(), row, v.data_ptr(), row, tokens, heads,
               kc.data_ptr(), vc.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    return kc, vc


def _without_allocation(k, v, row, tokens, heads):
    kc = torch.full((heads, 128), float("nan"), dtype=torch.float16, device=k.device)
    vc = torch.full_like(kc, float("nan"))
    _capi.call("pg_token_major_centers_noalloc", k.data_ptr(), row, v.data_ptr(), row, tokens,
               heads, kc.data_ptr(), vc.data_ptr(), _stream())
    return kc, vc


def test_noalloc_centers_equal_the_workspace_entry_point(cuda):
    lib = _capi.library()
    assert lib.pg_token_major_centers_noalloc_max_bytes() == 8 << 20
    # largest first (exactly the scratch bound: 512 chunks x 8 heads), then smaller
    cases = [(32768, 8, 0), (16384 + 37, 8, 3 * 128), (1000, 8, 0), (65, 2, 0), (1, 1, 0)]
    for i, (tokens, heads, pad) in enumerate(cases):
        print("noalloc case", tokens, heads, pad, flush=True)
        k, v, row = _inputs(tokens, heads, 20260850 + i, cuda, pad)
        want_k, want_v = _with_workspace(k, v, row, tokens, heads)
        got_k, got_v = _without_allocation(k, v, row, tokens, heads)
        torch.cuda.synchronize()
        assert torch.equal(got_k.view(torch.int16), want_k.view(torch.int16)), (tokens, heads)
        assert torch.equal(got_v.view(torch.int16), want_v.view(torch.int16)), (tokens, heads)


def test_noalloc_centers_reject_calls_beyond_the_scratch(cuda):
    lib = _capi.library()
    fake = 0x1000     # never dereferenced: the size check fails first
    rc = lib.pg_token_major_centers_noalloc(fake, 8 * 128, fake, 8 * 128, 32768 + 64, 8, fake,
                                            fake, _stream())
    assert rc == 4 and "at most 8 MiB" in _capi.last_error()
    # the failed call left the scratch usable
    k, v, row = _inputs(640, 4, 7, cuda)
    want = _with_workspace(k, v, row, 640, 4)
    got = _without_allocation(k, v, row, 640, 4)
    torch.cuda.synchronize()
    assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(got, want))


def test_noalloc_centers_check_their_pointers(cuda):
    rc = _capi.library().pg_token_major_centers_noalloc(None, 1024, None, 1024, 16, 8, None, None,
                                                         _stream())
    assert rc == 1 and "null tensor pointer" in _capi.last_error()


def test_noalloc_centers_replay_in_a_graph(cuda):
    """The caller this entry point is for: code under HIP graph capture.  One
    eager call first (it resolves this GPU's scratch address outside the
    capture), then the call captured on a side stream and replayed three
    times, each time after new K/V were copied into the captured buffers and
    with eager work (the workspace entry point on the same inputs) between
    the replays; every replay equals the workspace entry point bit for bit."""
    lib = _capi.library()
    tokens, heads = 4096 + 13, 8
    k, v, row = _inputs(tokens, heads, 11, cuda)
    kc = torch.full((heads, 128), float("nan"), dtype=torch.float16, device=cuda)
    vc = torch.full_like(kc, float("nan"))

    def call(stream):
        return lib.pg_token_major_centers_noalloc(k.data_ptr(), row, v.data_ptr(), row, tokens,
                                                  heads, kc.data_ptr(), vc.data_ptr(), stream)

    assert call(_stream()) == 0, _capi.last_error()          # warm-up, eager
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        rc = call(torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _capi.last_error()
    torch.cuda.synchronize()
    for replay in range(3):
        nk, nv, _ = _inputs(tokens, heads, 100 + replay, cuda)
        k.copy_(nk)
        v.copy_(nv)
        kc.fill_(float("nan"))
        vc.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_k, want_v = _with_workspace(k, v, row, tokens, heads)   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(kc.view(torch.int16), want_k.view(torch.int16)), replay
        assert torch.equal(vc.view(torch.int16), want_v.view(torch.int16)), replay
