"""Shared helpers of the test suite (CPU copies, oracle calls)."""

from __future__ import annotations

import numpy as np

from oracle import pg_oracle as oracle


def cpu(tensor) -> np.ndarray:
    return tensor.detach().cpu().numpy()


def bits(array: np.ndarray) -> np.ndarray:
    """Byte view for bit-exact comparisons (NaN payloads and -0 included)."""
    return np.ascontiguousarray(array).view(np.uint8)


def assert_bit_equal(got, want, what: str = "") -> None:
    got = cpu(got) if not isinstance(got, np.ndarray) else got
    if got.shape != want.shape or not np.array_equal(bits(got), bits(want)):
        diff = np.flatnonzero(bits(got).ravel() != bits(want).ravel())
        raise AssertionError(f"{what}: {diff.size} differing bytes (first at {diff[:5]})")


def oracle_decode(w, with_tail: bool = True, with_center: bool = True):
    """Oracle (float64) decode of a ``pagegauge_amd.workloads.DecodeWorkload``."""
    kw = {}
    if with_tail:
        kw.update(tail_k=cpu(w.tail_k), tail_v=cpu(w.tail_v), tail_indptr=cpu(w.tail_indptr),
                  tail_indices=cpu(w.tail_indices), tail_last_page_len=cpu(w.tail_last_page_len))
    if with_center:
        kw["value_center"] = cpu(w.value_center)
    return oracle.decode(cpu(w.query), cpu(w.k_codes), cpu(w.v_codes), cpu(w.old_indptr),
                         cpu(w.old_indices), cpu(w.old_last_page_len), w.sm_scale,
                         k_scale=cpu(w.k_scale), v_scale=cpu(w.v_scale), **kw)


def fp16_parity(out, ref16, ref64, tol: float = 2e-3) -> dict:
    """The 2e-3 bar for an FP16 attention output against the float64 oracle.

    ``ref16`` is the oracle rounded to FP16 (what the reference's own path
    returns), ``ref64`` the unrounded oracle.  An element passes when it is
    within ``tol`` of ``ref16``, or when it is the FP16 rounding of some value
    within ``tol`` of ``ref64`` (the distance from ``ref64`` to the interval
    of reals that round to it is at most ``tol``).  The second clause admits
    the other neighbour of a value that lies on a rounding midpoint: past
    |x| = 4 one FP16 ulp is already 3.9e-3, so a kernel exact to 1e-7 could
    otherwise fail by the rounding alone.  Returns the worst difference to
    ``ref16``, how many elements passed only by the second clause, and the
    worst distance to the rounding interval; ``ok`` is whether all passed."""
    got16 = (cpu(out) if not isinstance(out, np.ndarray) else out).astype(np.float16)
    got = got16.astype(np.float64)
    r16 = np.asarray(ref16).astype(np.float64)
    r64 = np.asarray(ref64).astype(np.float64)
    up = np.nextafter(got16, np.float16(np.inf)).astype(np.float64)
    down = np.nextafter(got16, np.float16(-np.inf)).astype(np.float64)
    # the reals that round to ``got``: half-way to each FP16 neighbour
    gap = np.where(r64 >= got, (r64 - got) - 0.5 * (up - got), (got - r64) - 0.5 * (got - down))
    d16 = np.abs(got - r16)
    near = d16 <= tol
    rounding = ~near & (gap <= tol)
    return {"max_fp16_diff": float(d16.max()), "boundary_flips": int(rounding.sum()),
            "max_interval_gap": float(np.maximum(gap, 0.0).max()),
            "ok": bool((near | rounding).all())}


def max_abs(a, b) -> float:
    a = cpu(a) if not isinstance(a, np.ndarray) else a
    b = cpu(b) if not isinstance(b, np.ndarray) else b
    return float(np.abs(a.astype(np.float64) - b.astype(np.float64)).max())


def dense_reference_class(dec, dtype=None, attention_output="kernel", tables="decoder"):
    """A ``dec.PageGaugeDecoder`` whose attention is the dense softmax, in
    ``dtype`` (float32 by default), over the reconstructed cache: K = c_K +
    s*Z for old pages and c_K + ring for tail pages, V likewise, from the same
    cache the K2 kernel updates (the reference's explicit-reconstruction path,
    diagnostics/benchmark_heterogeneous_fa2_correctness.py:291-299).  The
    PageGauge kernel runs on the same inputs first (it also finalizes a page
    that the step's token completes); ``kernel_error`` records max |kernel -
    dense| minus half an FP16 ulp of the dense value (the kernel's output
    rounding).  One request (batch 1).

    ``attention_output``: "kernel" feeds the FP16-rounded dense attention to
    the decoder's own O projection; "float16" and "float32" instead run the O
    projection as one float32 torch product of the FP16-rounded, or unrounded,
    dense attention (same epilogue: the projection rounded to FP16, then the
    FP16 residual add).  The two differ only by the FP16 rounding of the
    attention output, which measures the decoder's rounding floor.

    ``tables``: "decoder" reads the context through the decoder's own segment
    tables; "logical" rebuilds it from the page classes instead (the pinned
    ``page_table`` partition and exact-slot functions: every logical page of
    the context once, from the INT8 pool or from its exact slot), so that a
    wrong table cannot agree with itself."""
    import math

    import torch

    dtype = torch.float32 if dtype is None else dtype

    class DenseReference(dec.PageGaugeDecoder):
        kernel_error = 0.0

        def attention(self, layer):
            kernel = super().attention(layer).float().clone()
            dense = self._dense(layer)
            excess = (kernel.to(dtype) - dense).abs() - dense.abs() * 2.0 ** -11
            self.kernel_error = max(self.kernel_error, float(excess.max()))
            self.last_dense = dense
            self.attention_output[layer].copy_(dense.to(torch.float16))
            return self.attention_output[layer]

        def _layer_fused(self, layer):
            if attention_output == "kernel":
                return super()._layer_fused(layer)
            if not self.fused_append:
                raise ValueError("the float O projection reference runs the fused cache update")
            cfg = self.config
            w = self.weights.layers[layer]
            qw = cfg.q_heads * 128
            self._qkv_append(layer)
            self.attention(layer)
            a = self.last_dense.float()
            if attention_output == "float16":
                a = a.half().float()
            proj = torch.matmul(a.view(self.batch_size, qw), w["o"].float().t())
            self._hidden.copy_(self._hidden + proj.half())
            dec.projection(w["gate_up"], self._hidden, self._activation,
                           norm_weight=w["post_norm"], eps=cfg.rms_eps, swiglu=True)
            dec.projection(w["down"], self._activation, self._hidden, residual=self._hidden)

        def _logical_tables(self, b):
            from pagegauge_amd import page_table as pt

            last = int(self.exact_table.host_last_len[b])
            pages = self.current_pages
            part = pt.page_gauge_logical_partition(
                pages, self.exact_tail_pages, self.exact_sink_pages, last,
                self.exact_static_suffix_pages, self.initial_context_pages)
            old = [b * self.max_pages + p for p in part["old_logical_pages"]]
            exact = [pt.exact_physical_page_index(b, p, self.exact_tail_pages,
                                                  self.exact_sink_pages,
                                                  self.exact_static_suffix_pages,
                                                  self.initial_context_pages)
                     for p in part["exact_logical_pages"]]
            assert part["exact_logical_pages"][-1] == pages - 1   # the newest page is exact
            device = self.cache.key_codes.device
            return (torch.tensor(old, device=device), torch.tensor(exact, device=device), last)

        def _dense(self, layer):
            c = self.cache
            b = 0
            if tables == "logical":
                old, tail, last = self._logical_tables(b)
            else:
                old = self.old_table.active_indices().long()
                tail = self.exact_table.active_indices().long()
                last = int(self.exact_table.host_last_len[b])
            kc = c.key_center[layer, b].to(dtype)
            vc = c.value_center[layer, b].to(dtype)
            k_old = c.key_codes[layer][old].to(dtype) * c.key_scales[layer][old].to(dtype)[:, None, :, None]
            v_old = c.value_codes[layer][old].to(dtype) * c.value_scales[layer][old].to(dtype)[:, None, :, None]
            k_tail = c.exact_key[layer][tail].to(dtype)
            v_tail = c.exact_value[layer][tail].to(dtype)
            n_tail = (tail.numel() - 1) * 16 + last
            keys = torch.cat((k_old.reshape(-1, 8, 128), k_tail.reshape(-1, 8, 128)[:n_tail])) + kc
            values = torch.cat((v_old.reshape(-1, 8, 128), v_tail.reshape(-1, 8, 128)[:n_tail])) + vc
            q = self.rotated_query[b].to(dtype).view(8, 4, 128)
            scores = torch.matmul(q, keys.permute(1, 2, 0).contiguous()) / math.sqrt(128)
            probs = torch.softmax(scores, dim=-1)
            return torch.matmul(probs, values.permute(1, 0, 2).contiguous()).reshape(1, 32, 128)

    return DenseReference
