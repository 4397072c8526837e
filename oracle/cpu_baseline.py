"""Torch-CPU restatement of the PageGauge decode path, for the CPU baseline.

TEST INFRASTRUCTURE ONLY (like the rest of ``oracle/``): ``bench.py``'s
CPU-baseline leg times it on the GPU box's host cores, and
``tests/test_oracle.py`` pins it against the numpy oracle.  The product
package never imports it.

The reference has no CPU path (its drivers exit without CUDA,
scripts/benchmark_flashinfer_page_affine_int8.py:425-426), so the CPU baseline
is this restatement of the reference formulas, written as a CPU implementation
would be (torch tensor ops on every host thread, float32 arithmetic):

* ``decode_dense``: the INT8 pages dequantised (code * page scale), the FP16
  tail ring appended, dense float32 softmax attention per request with the
  GQA group of 4, the value center added, and the base-2 LSE
  (scripts/benchmark_flashinfer_page_affine_int8.py:566-602; the tail merge of
  tests/page_gauge_append_extension.cu:389-583 is the same softmax);
* ``append_positions``: RoPE, centered append into the ring and the completed
  page's INT8 finalize, one position per request
  (tests/page_gauge_append_extension.cu:148-383, per-request positions as the
  Triton append_finalize_page_gauge, scripts/benchmark_page_gauge_overheads.py:112-205);
* ``CpuDecoder``: one Mistral-architecture decoder step over a PageGauge
  cache filled with random K/V, as the reference's own decoder benchmark
  fills its caches (scripts/benchmark_page_gauge_transformer.py:1156-1259),
  every layer's attention through ``decode_dense`` and the new token through
  ``append_positions``.
"""

from __future__ import annotations

import torch

PAGE = 16
DIM = 128
GQA = 4
LOG2E = 1.4426950408889634


# ---------------------------------------------------------------------------
# Decode (A4/A5)
# ---------------------------------------------------------------------------

def _gather(pages: torch.Tensor, scale, indptr, indices, last_page_len, request: int):
    """One request's tokens [T, Hkv, 128] in float32 (dequantised when
    ``scale`` is given)."""
    begin, end = int(indptr[request]), int(indptr[request + 1])
    if end <= begin:
        return pages.new_zeros((0, pages.shape[2], DIM), dtype=torch.float32)
    ids = indices[begin:end].long()
    block = pages.index_select(0, ids).float()                   # [n, 16, Hkv, 128]
    if scale is not None:
        block = block * scale.index_select(0, ids).float()[:, None, :, None]
    n = ids.numel()
    return block.reshape(n * PAGE, pages.shape[2], DIM)[: (n - 1) * PAGE + int(last_page_len[request])]


def decode_dense(query, k_pages, v_pages, indptr, indices, last_page_len, sm_scale: float,
                 k_scale=None, v_scale=None, tail_k=None, tail_v=None, tail_indptr=None,
                 tail_indices=None, tail_last_page_len=None, value_center=None):
    """Dense float32 paged decode; arguments as ``pg_oracle.decode`` (torch
    CPU tensors).  Returns (out float16 [B, Hq, 128], lse float32 [B, Hq])."""
    batch, hq, _ = query.shape
    hkv = k_pages.shape[2]
    out = torch.empty(batch, hq, DIM, dtype=torch.float16)
    lse = torch.empty(batch, hq, dtype=torch.float32)
    for request in range(batch):
        keys = _gather(k_pages, k_scale, indptr, indices, last_page_len, request)
        values = _gather(v_pages, v_scale, indptr, indices, last_page_len, request)
        if tail_k is not None:
            keys = torch.cat((keys, _gather(tail_k, None, tail_indptr, tail_indices,
                                            tail_last_page_len, request)))
            values = torch.cat((values, _gather(tail_v, None, tail_indptr, tail_indices,
                                                tail_last_page_len, request)))
        q = query[request].float().view(hkv, hq // hkv, DIM)
        scores = torch.matmul(q, keys.permute(1, 2, 0)) * sm_scale      # [Hkv, G, T]
        if keys.shape[0] == 0:
            o = torch.zeros(hkv, hq // hkv, DIM)
            row_lse = torch.full((hkv, hq // hkv), float("-inf"))
        else:
            row_lse = torch.logsumexp(scores, dim=-1)
            probs = torch.exp(scores - row_lse[..., None])
            o = torch.matmul(probs, values.permute(1, 0, 2))             # [Hkv, G, 128]
        if value_center is not None:
            center = value_center if value_center.dim() == 2 else value_center[request]
            o = o + center.float()[:, None, :]
        out[request] = o.reshape(hq, DIM).to(torch.float16)
        lse[request] = (row_lse * LOG2E).reshape(hq)
    return out, lse


# ---------------------------------------------------------------------------
# Cache update (A1-A3), one position per request
# ---------------------------------------------------------------------------

def rope(x: torch.Tensor, cosine: torch.Tensor, sine: torch.Tensor) -> torch.Tensor:
    """HF RoPE in FP16 tensor ops: x*cos + rotate_half(x)*sin, each product
    and the sum rounded to FP16 (the products of two halves are exact in
    float32, and a float32 sum of two halves rounds to FP16 as a direct
    rounding would)."""
    partner = torch.cat((-x[..., DIM // 2:], x[..., :DIM // 2]), dim=-1)
    return (x * cosine).to(torch.float16) + (partner * sine).to(torch.float16)


def finalize(page: torch.Tensor):
    """Codes and scale of completed ring pages [..., 16, 128] (FP16): per
    block, s = fp16(max(amax/127, 2^-20)), codes = sign-symmetric
    floor(q + 0.5) of the float32 quotient, clamped to [-127, 127]."""
    values = page.float()
    amax = values.abs().amax(dim=(-2, -1), keepdim=True)
    scale = torch.clamp(amax / 127.0, min=2.0 ** -20).to(torch.float16)
    quotient = values / scale.float()
    magnitude = torch.floor(quotient.abs() + 0.5)
    codes = torch.clamp(torch.copysign(magnitude, quotient), -127, 127).to(torch.int8)
    return codes, scale[..., 0, 0]


def append_positions(query, key, value, cos_table, sin_table, positions, key_center,
                     value_center, rotated_query, exact_k, exact_v, codes_k, codes_v, scales_k,
                     scales_v, sink_pages: int = 0) -> None:
    """In place: rotate the queries, write each request's centered K/V row
    into its ring slot and finalize a page on its 16th token.  Pools are
    request-major: ring pages [B*E, 16, Hkv, 128], code pages [B*P, ...]."""
    batch, hkv = key.shape[0], key.shape[1]
    ring_pages = exact_k.shape[0] // batch
    code_pages = codes_k.shape[0] // batch
    pos = positions.long()
    cos, sin = cos_table[pos].to(torch.float16), sin_table[pos].to(torch.float16)
    rotated_query.copy_(rope(query, cos[:, None, :], sin[:, None, :]))
    rotated_key = rope(key, cos[:, None, :], sin[:, None, :])
    kc = key_center if key_center.dim() == 3 else key_center.expand(batch, hkv, DIM)
    vc = value_center if value_center.dim() == 3 else value_center.expand(batch, hkv, DIM)
    ring_row_k = (rotated_key.float() - kc.float()).to(torch.float16)
    ring_row_v = (value.float() - vc.float()).to(torch.float16)
    tail = ring_pages - sink_pages
    for r in range(batch):
        page, token = divmod(int(pos[r]), PAGE)
        if page >= code_pages:
            continue
        local = page if page < sink_pages else sink_pages + page % tail
        slot = r * ring_pages + local
        exact_k[slot, token] = ring_row_k[r]
        exact_v[slot, token] = ring_row_v[r]
        if token == PAGE - 1:
            code_page = r * code_pages + page
            for ring, codes, scales in ((exact_k, codes_k, scales_k), (exact_v, codes_v, scales_v)):
                block = ring[slot].permute(1, 0, 2)                  # [Hkv, 16, 128]
                c, s = finalize(block)
                codes[code_page] = c.permute(1, 0, 2)
                scales[code_page] = s


# ---------------------------------------------------------------------------
# Decoder step
# ---------------------------------------------------------------------------

class CpuDecoder:
    """Mistral-architecture decoder (float32 weights) over a PageGauge cache
    of ``context`` tokens per layer, filled with random K/V (INT8 history
    pages through ``finalize``, the newest ``tail_pages`` pages as the exact
    ring).  ``layers`` may be fewer than the model's (a stated cap)."""

    def __init__(self, layers: int, context: int, seed: int, hidden: int = 4096,
                 q_heads: int = 32, kv_heads: int = 8, intermediate: int = 14336,
                 vocab: int = 32768, tail_pages: int = 16, steps: int = 16,
                 theta: float = 1.0e6, eps: float = 1.0e-5, std: float = 0.02) -> None:
        gen = torch.Generator().manual_seed(seed)
        normal = lambda *shape: torch.randn(*shape, generator=gen) * std  # noqa: E731
        self.hidden, self.q_heads, self.kv_heads = hidden, q_heads, kv_heads
        self.intermediate, self.eps = intermediate, eps
        self.embed = normal(vocab, hidden)
        self.lm_head = normal(vocab, hidden)
        self.layers = [{"qkv": normal((q_heads + 2 * kv_heads) * DIM, hidden),
                        "o": normal(hidden, hidden), "gate_up": normal(2 * intermediate, hidden),
                        "down": normal(hidden, intermediate)} for _ in range(layers)]
        inv = 1.0 / (theta ** (torch.arange(0, DIM, 2).float() / DIM))
        freqs = torch.arange(context + steps + 1).float()[:, None] * inv[None]
        emb = torch.cat((freqs, freqs), dim=-1)
        self.cos, self.sin = emb.cos().half(), emb.sin().half()
        self.tail_pages = tail_pages
        code_pages = -(-(context + steps + 1) // PAGE)
        old_pages = context // PAGE - tail_pages
        self.cache = []
        for _ in range(layers):
            keys = torch.randn(context, kv_heads, DIM, generator=gen).half()
            values = torch.randn(context, kv_heads, DIM, generator=gen).half()
            kc, vc = keys.float().mean(0).half(), values.float().mean(0).half()
            ck = (keys.float() - kc.float()).half().view(-1, PAGE, kv_heads, DIM)
            cv = (values.float() - vc.float()).half().view(-1, PAGE, kv_heads, DIM)
            layer = {"key_center": kc, "value_center": vc,
                     "codes_k": torch.zeros(code_pages, PAGE, kv_heads, DIM, dtype=torch.int8),
                     "codes_v": torch.zeros(code_pages, PAGE, kv_heads, DIM, dtype=torch.int8),
                     "scales_k": torch.zeros(code_pages, kv_heads, dtype=torch.float16),
                     "scales_v": torch.zeros(code_pages, kv_heads, dtype=torch.float16),
                     "exact_k": torch.zeros(tail_pages, PAGE, kv_heads, DIM, dtype=torch.float16),
                     "exact_v": torch.zeros(tail_pages, PAGE, kv_heads, DIM, dtype=torch.float16)}
            # every complete prompt page has codes (the cache update finalized
            # it when its 16th token landed); the newest pages are also in the ring
            whole = context // PAGE
            for src, codes, scales in ((ck, layer["codes_k"], layer["scales_k"]),
                                       (cv, layer["codes_v"], layer["scales_v"])):
                c, s = finalize(src.permute(0, 2, 1, 3))
                codes[:whole] = c.permute(0, 2, 1, 3)
                scales[:whole] = s
            for p in range(old_pages, context // PAGE):
                layer["exact_k"][p % tail_pages] = ck[p]
                layer["exact_v"][p % tail_pages] = cv[p]
            self.cache.append(layer)

    def _rms(self, x: torch.Tensor) -> torch.Tensor:
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)

    def step(self, token: int, position: int) -> torch.Tensor:
        """Logits [vocab] of ``token`` at ``position`` (the cache holds
        ``position`` tokens); appends its K/V."""
        qw, kw = self.q_heads * DIM, self.kv_heads * DIM
        x = self.embed[token][None]
        pages = position // PAGE + 1
        old = max(pages - self.tail_pages, 0)
        i32 = lambda v: torch.tensor(v, dtype=torch.int32)  # noqa: E731
        old_indptr, old_indices = i32([0, old]), torch.arange(old, dtype=torch.int32)
        tail_indptr = i32([0, pages - old])
        tail_indices = i32([p % self.tail_pages for p in range(old, pages)])
        last = i32([PAGE])
        tail_last = i32([position % PAGE + 1])
        for w, c in zip(self.layers, self.cache):
            qkv = self._rms(x) @ w["qkv"].t()
            q = qkv[:, :qw].view(1, self.q_heads, DIM).half()
            k = qkv[:, qw:qw + kw].view(1, self.kv_heads, DIM).half()
            v = qkv[:, qw + kw:].view(1, self.kv_heads, DIM).half()
            rq = torch.empty_like(q)
            append_positions(q, k, v, self.cos, self.sin, i32([position]), c["key_center"],
                             c["value_center"], rq, c["exact_k"], c["exact_v"], c["codes_k"],
                             c["codes_v"], c["scales_k"], c["scales_v"])
            attn, _ = decode_dense(rq, c["codes_k"], c["codes_v"], old_indptr, old_indices, last,
                                   DIM ** -0.5, k_scale=c["scales_k"], v_scale=c["scales_v"],
                                   tail_k=c["exact_k"], tail_v=c["exact_v"],
                                   tail_indptr=tail_indptr, tail_indices=tail_indices,
                                   tail_last_page_len=tail_last, value_center=c["value_center"])
            x = x + attn.float().view(1, qw) @ w["o"].t()
            gate, up = (self._rms(x) @ w["gate_up"].t()).split(self.intermediate, dim=-1)
            x = x + (torch.nn.functional.silu(gate) * up) @ w["down"].t()
        return (self._rms(x) @ self.lm_head.t())[0]


def host_description() -> dict:
    """CPU model, logical CPUs and torch's thread count of this host."""
    import os
    import platform

    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


__all__ = ["CpuDecoder", "append_positions", "decode_dense", "finalize", "host_description",
           "rope"]
