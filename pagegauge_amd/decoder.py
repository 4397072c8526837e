"""Mistral-architecture decoder whose KV cache and attention run on PageGauge.

The caller of the hot path: ``TransformerDecoder`` / ``GaugeCache`` /
``GraphDecodeWrapper`` of scripts/benchmark_page_gauge_transformer.py
(:321-380, :1262-1580, :1583-2330, :2754-2805, :3159-3275) and the prefill
cache population of diagnostics/benchmark_backend_exclusive.py:372-506.

Per decode step and layer (``_layer``):
  RMSNorm -> fused QKV projection -> K2 (``rope_append_page_gauge_dynamic``:
  RoPE, centered append into the FP16 ring, INT8 finalize of a completed page)
  -> K1 (``PageGaugeSegmentedDecode``: INT8 history + FP16 tail + value
  center, one partial kernel and one combine kernel) -> output projection ->
  residual -> RMSNorm -> fused gate/up -> SiLU * up -> down -> residual.

Everything but K1/K2 is plain PyTorch-ROCm (fp16 GEMMs on hipBLASLt).  The
``"fp16"`` backend is the same decoder over an FP16 paged cache
(``rope_append_fp16_dynamic`` + the same-way FP16 decode kernel): the
reference's ``flashinfer_fp16`` baseline.

A decode step can be captured as ONE HIP graph (embedding, 32 layers, final
norm, LM head, greedy argmax) that reads the position from a device scalar,
so the 16 steps of one page window replay the same graph.  Graphs are banked
by the structural plan signature; ``plan`` re-plans the split-KV work list
only when that signature changes (``SegmentTable``).

Weights are random-init (normal(0, 0.02), norms one: the HF initializer of
``MistralForCausalLM``), generated on the device from a seed; there are no
checkpoints here.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Optional

import torch
import torch.nn.functional as F

from . import page_table as pt
from .decode import (BatchDecodeWithPagedKVCacheWrapper, HeterogeneousDecodeWrapper,
                     PageGaugeSegmentedDecode)
from .runtime import load_append_extension
from .update import prefill_page_gauge, token_major_centers

PAGE = 16
DIM = 128
GQA = 4


@dataclass(frozen=True)
class DecoderConfig:
    """Mistral-7B-v0.3 architecture by default."""

    layers: int = 32
    hidden: int = 4096
    q_heads: int = 32
    kv_heads: int = 8
    intermediate: int = 14336
    vocab: int = 32768
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-5
    init_std: float = 0.02

    def __post_init__(self) -> None:
        if self.q_heads * DIM != self.hidden or self.q_heads != GQA * self.kv_heads:
            raise ValueError("the decode kernels need head_dim 128 and GQA group 4")
        if self.layers <= 0 or self.intermediate <= 0 or self.vocab <= 0:
            raise ValueError("layers, intermediate size and vocabulary must be positive")

    @property
    def qkv_width(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * DIM


def rope_tables(positions: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """HF rotary tables [positions, 128] FP16, computed in float32 on the CPU
    (``model.model.rotary_emb`` then ``.to(float16)``,
    scripts/benchmark_page_gauge_transformer.py:3628-3636)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, DIM, 2, dtype=torch.int64).float() / DIM))
    t = torch.arange(positions, dtype=torch.int64).float()
    freqs = t[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.float16).contiguous(), emb.sin().to(torch.float16).contiguous()


class DecoderWeights:
    """Random-init FP16 weights with fused QKV and gate/up projections (the
    packing of ``BASE_E2E.pack_model_projections``)."""

    def __init__(self, config: DecoderConfig, seed: int, device="cuda") -> None:
        self.config = config
        gen = torch.Generator(device=device).manual_seed(seed)
        std = config.init_std

        def normal(*shape):
            w = torch.empty(*shape, device=device, dtype=torch.float16)
            return w.normal_(0.0, std, generator=gen)

        h, i = config.hidden, config.intermediate
        self.embed = normal(config.vocab, h)
        self.layers = []
        for _ in range(config.layers):
            self.layers.append({
                "input_norm": torch.ones(h, device=device, dtype=torch.float16),
                "qkv": normal(config.qkv_width, h),
                "o": normal(h, h),
                "post_norm": torch.ones(h, device=device, dtype=torch.float16),
                "gate_up": normal(2 * i, h),
                "down": normal(h, i),
            })
        self.norm = torch.ones(h, device=device, dtype=torch.float16)
        self.lm_head = normal(config.vocab, h)

    def bytes_per_token(self) -> int:
        """Weight bytes streamed by one decode step (embedding row excluded)."""
        per_layer = sum(w.numel() * w.element_size() for w in self.layers[0].values())
        return self.config.layers * per_layer + self.lm_head.numel() * 2 + self.norm.numel() * 2


def projection(weight: torch.Tensor, x: torch.Tensor, out: torch.Tensor, *,
               norm_weight: Optional[torch.Tensor] = None, eps: float = 1.0e-5,
               swiglu: bool = False, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``out = epilogue(weight @ prologue(x))`` in one HIP launch
    (``pg_decoder_gemv``).  Prologue: MistralRMSNorm with ``norm_weight``, or
    nothing.  Epilogue: the projection rounded to FP16; with ``swiglu`` the
    weight rows are [gate; up] and ``out[i] = silu(gate_i) * up_i`` (FP16
    ops, ``out`` has N/2 columns); then ``residual`` added in FP16
    (``residual`` may be ``out``).  ``out`` is FP16 or float32 [B, N']."""
    from . import _capi

    n, k = int(weight.shape[0]), int(weight.shape[1])
    batch = int(x.shape[0])
    if weight.dtype != torch.float16 or not weight.is_contiguous() or x.dtype != torch.float16:
        raise ValueError("projection weights and inputs must be FP16 (weights contiguous)")
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] != k:
        raise ValueError("projection input must be [B, K] rows")
    width = n // 2 if swiglu else n
    if out.dim() != 2 or tuple(out.shape) != (batch, width) or out.stride(1) != 1:
        raise ValueError("projection output must be [B, N] rows ([B, N/2] with SwiGLU)")
    if residual is not None and (tuple(residual.shape) != (batch, width) or residual.stride(1) != 1
                                 or residual.dtype != torch.float16):
        raise ValueError("residual must be FP16 rows shaped like the output")
    if norm_weight is not None and (norm_weight.numel() != k or norm_weight.dtype != torch.float16):
        raise ValueError("norm weight must be FP16 [K]")
    out_f32 = out.dtype == torch.float32
    if not out_f32 and out.dtype != torch.float16:
        raise ValueError("projection output must be FP16 or float32")
    _capi.call("pg_decoder_gemv", weight.data_ptr(), n, k, x.data_ptr(), x.stride(0), batch,
               None if norm_weight is None else norm_weight.data_ptr(), float(eps), int(swiglu),
               None if residual is None else residual.data_ptr(),
               0 if residual is None else residual.stride(0), out.data_ptr(), out.stride(0),
               int(out_f32), torch.cuda.current_stream().cuda_stream)
    return out


def qkv_rope_append(weight: torch.Tensor, x: torch.Tensor, *, norm_weight: torch.Tensor,
                    eps: float, query_heads: int, kv_heads: int, cos: torch.Tensor,
                    sin: torch.Tensor, positions: torch.Tensor, rotated_query: torch.Tensor,
                    key_pages: torch.Tensor, value_pages: torch.Tensor,
                    key_center: Optional[torch.Tensor], value_center: Optional[torch.Tensor],
                    pages_per_request: int, sink_pages: int, capacity_tokens: int) -> None:
    """The QKV projection fused with the decode step's cache update
    (``pg_decoder_qkv_rope_append``): RMSNorm, QKV rows, RoPE of query and
    key, and the (centered, with ``key_center``) append of key and value at
    ``positions`` (device int32, one shared or one per row) -- bit-identical to
    ``projection`` followed by ``rope_append_page_gauge_dynamic`` /
    ``rope_append_fp16_dynamic``, except that the PageGauge page finalize is
    left to the decode (``finalize=`` of its run)."""
    from . import _capi

    batch, k = int(x.shape[0]), int(x.shape[1])
    rows = (query_heads + 2 * kv_heads) * DIM
    if (weight.dtype != torch.float16 or not weight.is_contiguous()
            or tuple(weight.shape) != (rows, k)):
        raise ValueError("QKV weights must be contiguous FP16 [(Hq + 2 Hkv) * 128, K]")
    if x.dtype != torch.float16 or x.stride(1) != 1:
        raise ValueError("projection input must be FP16 [B, K] rows")
    for t, name in ((cos, "cos"), (sin, "sin"), (rotated_query, "rotated_query"),
                    (key_pages, "key_pages"), (value_pages, "value_pages")):
        if t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous FP16")
    if positions.dtype != torch.int32 or positions.numel() not in (1, batch):
        raise ValueError("positions must be int32, one shared or one per row")
    tensors = (weight, x, norm_weight, cos, sin, positions, rotated_query, key_pages, value_pages)
    if not all(t.is_cuda and t.device == weight.device for t in tensors):
        raise ValueError("all tensors must be on the weights' CUDA device")
    if norm_weight.dtype != torch.float16 or norm_weight.numel() != k:
        raise ValueError("norm weight must be FP16 [K]")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != DIM:
        raise ValueError("RoPE tables must be matching [positions, 128] tensors")
    if tuple(rotated_query.shape) != (batch, query_heads, DIM):
        raise ValueError("rotated_query must be [B, Hq, 128]")
    if (key_pages.shape != value_pages.shape or key_pages.dim() != 4
            or tuple(key_pages.shape[1:]) != (PAGE, kv_heads, DIM)
            or key_pages.shape[0] < batch * pages_per_request):
        raise ValueError("key/value pages must be [>= B * pages_per_request, 16, Hkv, 128]")
    if key_center is None:
        if value_center is not None or capacity_tokens > pages_per_request * PAGE:
            raise ValueError("FP16 pages: no centers, capacity within pages_per_request pages")
    else:
        for center in (key_center, value_center):
            if (center is None or center.dtype != torch.float16 or not center.is_contiguous()
                    or tuple(center.shape[-2:]) != (kv_heads, DIM)
                    or center.numel() != batch * kv_heads * DIM):
                raise ValueError("centers must be contiguous FP16 [B, Hkv, 128]")
        if not 0 <= sink_pages < pages_per_request:
            raise ValueError("the exact ring needs at least one tail page after the sink")
    stride = 1 if positions.numel() == batch and batch > 1 else 0
    center_stride = 0 if key_center is None else kv_heads * DIM
    _capi.call("pg_decoder_qkv_rope_append", weight.data_ptr(), k, x.data_ptr(), x.stride(0),
               batch, norm_weight.data_ptr(), float(eps), query_heads, kv_heads, cos.data_ptr(),
               sin.data_ptr(), cos.stride(0), int(cos.shape[0]), positions.data_ptr(), stride,
               rotated_query.data_ptr(), key_pages.data_ptr(), value_pages.data_ptr(),
               None if key_center is None else key_center.data_ptr(),
               None if value_center is None else value_center.data_ptr(), center_stride,
               int(pages_per_request), int(sink_pages), int(capacity_tokens),
               torch.cuda.current_stream().cuda_stream)


def argmax_rows(x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``torch.argmax(x, dim=-1, out=out)`` for float32 logits [B, V] in one
    HIP launch (``pg_argmax_f32``): the first index of the maximum, NaN
    counting as the largest value."""
    from . import _capi

    if x.dtype != torch.float32 or x.dim() != 2 or x.stride(1) != 1 or not x.is_cuda:
        raise ValueError("argmax input must be CUDA float32 [B, V] rows")
    if out.dtype != torch.int64 or out.numel() != x.shape[0] or not out.is_contiguous():
        raise ValueError("argmax output must be contiguous int64 [B]")
    _capi.call("pg_argmax_f32", x.data_ptr(), int(x.shape[0]), int(x.shape[1]), x.stride(0),
               out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """MistralRMSNorm: float32 statistics, FP16 product with the weight."""
    x32 = x.float()
    x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    return weight * x32.to(x.dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin in FP16 tensor ops (each op rounds to
    FP16, the arithmetic of the K2 kernel).  x [T, H, 128], cos/sin [T, 128]."""
    rotated = torch.cat((-x[..., DIM // 2:], x[..., :DIM // 2]), dim=-1)
    return x * cos[:, None, :] + rotated * sin[:, None, :]


def _causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      chunk: int = 1024) -> torch.Tensor:
    """Prefill attention, [T,Hq,128] x [T,Hkv,128] -> [T,Hq,128] FP16.

    Query heads 4g..4g+3 share KV head g, so a block of queries is laid out
    [Hkv, 4*chunk, 128] and multiplied by contiguous K^T [Hkv, 128, T]; the
    softmax is float32.  Memory is bounded by the query chunk."""
    tokens, hq, _ = q.shape
    hkv = k.shape[1]
    scale = 1.0 / math.sqrt(DIM)
    kt = k.permute(1, 2, 0).contiguous()            # [Hkv, 128, T]
    vh = v.permute(1, 0, 2).contiguous()            # [Hkv, T, 128]
    out = torch.empty_like(q)
    for begin in range(0, tokens, chunk):
        end = min(tokens, begin + chunk)
        n = end - begin
        qc = q[begin:end].view(n, hkv, GQA, DIM).permute(1, 2, 0, 3).reshape(hkv, GQA * n, DIM)
        scores = torch.matmul(qc.contiguous(), kt[:, :, :end]).float() * scale   # [Hkv, 4n, end]
        rows = torch.arange(begin, end, device=q.device).repeat(GQA)
        mask = torch.arange(end, device=q.device)[None, :] > rows[:, None]
        scores.masked_fill_(mask[None], float("-inf"))
        probs = torch.softmax(scores, dim=-1).to(v.dtype)
        o = torch.matmul(probs, vh[:, :end])          # [Hkv, 4n, 128]
        out[begin:end] = o.view(hkv, GQA, n, DIM).permute(2, 0, 1, 3).reshape(n, hq, DIM)
    return out


@torch.inference_mode()
def prefill(weights: DecoderWeights, tokens: torch.Tensor, cos: torch.Tensor,
            sin: torch.Tensor, on_layer=None) -> torch.Tensor:
    """Run a B=1 prompt [T] through the model; returns the last position's
    float32 logits [1, vocab].  ``on_layer(layer, key, value)`` receives each
    layer's rotated keys and values [T, Hkv, 128] (FP16, views valid only
    during the call) to populate the caches."""
    cfg = weights.config
    tokens = tokens.reshape(-1)
    count = tokens.numel()
    hidden = F.embedding(tokens, weights.embed)
    c, s = cos[:count], sin[:count]
    qw, kw = cfg.q_heads * DIM, cfg.kv_heads * DIM
    for index, w in enumerate(weights.layers):
        x = rms_norm(hidden, w["input_norm"], cfg.rms_eps)
        qkv = F.linear(x, w["qkv"])
        q = rope(qkv[:, :qw].view(count, cfg.q_heads, DIM), c, s)
        k = rope(qkv[:, qw:qw + kw].view(count, cfg.kv_heads, DIM), c, s)
        v = qkv[:, qw + kw:].view(count, cfg.kv_heads, DIM)
        if on_layer is not None:
            on_layer(index, k, v)
        attn = _causal_attention(q, k, v)
        hidden = hidden + F.linear(attn.reshape(count, qw), w["o"])
        x = rms_norm(hidden, w["post_norm"], cfg.rms_eps)
        gate, up = F.linear(x, w["gate_up"]).split(cfg.intermediate, dim=-1)
        hidden = hidden + F.linear(F.silu(gate) * up, w["down"])
        del qkv, q, k, v, attn, x, gate, up
    last = rms_norm(hidden[-1:], weights.norm, cfg.rms_eps)
    return F.linear(last, weights.lm_head).float()


# ---------------------------------------------------------------------------
# Caches
# ---------------------------------------------------------------------------

class Fp16Cache:
    """Request-major FP16 paged cache [L, B*P, 16, Hkv, 128] (``BaselineCache``)."""

    def __init__(self, config: DecoderConfig, batch_size: int, pages: int, device="cuda") -> None:
        shape = (config.layers, batch_size * pages, PAGE, config.kv_heads, DIM)
        self.key = torch.zeros(shape, device=device, dtype=torch.float16)
        self.value = torch.zeros_like(self.key)
        self.pages_per_request = pages

    def clone(self) -> "Fp16Cache":
        other = Fp16Cache.__new__(Fp16Cache)
        other.key, other.value = self.key.clone(), self.value.clone()
        other.pages_per_request = self.pages_per_request
        return other

    def populate(self, layer: int, request: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Write a token-major prefix [T, Hkv, 128] (T a multiple of 16)."""
        pages = key.shape[0] // PAGE
        base = request * self.pages_per_request
        self.key[layer, base:base + pages].copy_(key.reshape(pages, PAGE, *key.shape[1:]))
        self.value[layer, base:base + pages].copy_(value.reshape(pages, PAGE, *value.shape[1:]))


class GaugeCache:
    """PageGauge storage (scripts/benchmark_page_gauge_transformer.py:321-380):
    INT8 codes [L, B*P, 16, Hkv, 128], scales [L, B*P, Hkv], per-request
    centers [L, B, Hkv, 128] and the exact FP16 pages [L, B*E, 16, Hkv, 128],
    E = S prefix (sink) pages + A static-suffix pages (the A pages before
    ``initial_context_pages``, kept exact for the whole decode) + the tail
    ring, in that order per request."""

    def __init__(self, config: DecoderConfig, batch_size: int, pages: int,
                 exact_tail_pages: int, exact_sink_pages: int = 0, device="cuda",
                 exact_static_suffix_pages: int = 0,
                 initial_context_pages: Optional[int] = None) -> None:
        layout = pt.ExactPageLayout.checked(exact_sink_pages, exact_static_suffix_pages,
                                            initial_context_pages, exact_tail_pages)
        if exact_tail_pages <= 0:
            raise ValueError("at least one tail-ring page is required")
        L, hkv = config.layers, config.kv_heads
        self.key_codes = torch.zeros(L, batch_size * pages, PAGE, hkv, DIM, device=device,
                                     dtype=torch.int8)
        self.value_codes = torch.zeros_like(self.key_codes)
        self.key_scales = torch.zeros(L, batch_size * pages, hkv, device=device, dtype=torch.float16)
        self.value_scales = torch.zeros_like(self.key_scales)
        self.key_center = torch.zeros(L, batch_size, hkv, DIM, device=device, dtype=torch.float16)
        self.value_center = torch.zeros_like(self.key_center)
        self.exact_tail_pages = exact_tail_pages
        self.exact_sink_pages = exact_sink_pages
        self.exact_static_suffix_pages = layout.suffix
        self.initial_context_pages = layout.initial
        self.exact_fixed_pages = layout.fixed
        self.exact_storage_pages_per_request = layout.storage
        ring = batch_size * self.exact_storage_pages_per_request
        self.exact_key = torch.zeros(L, ring, PAGE, hkv, DIM, device=device, dtype=torch.float16)
        self.exact_value = torch.zeros_like(self.exact_key)
        self.pages_per_request = pages
        self.batch_size = batch_size
        self._center_workspace: Optional[torch.Tensor] = None

    def clone(self) -> "GaugeCache":
        other = GaugeCache.__new__(GaugeCache)
        for name, value in vars(self).items():
            setattr(other, name, value.clone() if isinstance(value, torch.Tensor) else value)
        other._center_workspace = None
        return other

    def populate(self, layer: int, request: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Cache a token-major prefix [T, Hkv, 128] of whole pages: exact
        centers, INT8 codes and scales of every page, and the centered FP16
        copies of its exact pages (the sink prefix, the static suffix and the
        last tail pages) in their slots
        (diagnostics/benchmark_backend_exclusive.py:427-506)."""
        tokens = key.shape[0]
        pages = tokens // PAGE
        if tokens % PAGE or pages > self.pages_per_request:
            raise ValueError("prefix must be whole pages within the cache capacity")
        if pages <= self.exact_tail_pages + self.exact_sink_pages:
            raise ValueError("fixture must contain at least one quantized old page")
        if self.exact_static_suffix_pages and pages < self.initial_context_pages:
            raise ValueError("the static suffix lies beyond the cached prefix")
        from . import _capi
        need = int(_capi.library().pg_token_major_centers_workspace_bytes(tokens, key.shape[1]))
        if self._center_workspace is None or self._center_workspace.numel() < need:
            self._center_workspace = torch.empty(need, device=key.device, dtype=torch.uint8)
        kc, vc = self.key_center[layer, request], self.value_center[layer, request]
        token_major_centers(key, value, kc, vc, self._center_workspace)
        exact_map = torch.full((pages,), -1, dtype=torch.int32)
        partition = pt.page_gauge_logical_partition(
            pages, self.exact_tail_pages, self.exact_sink_pages, PAGE,
            self.exact_static_suffix_pages, self.initial_context_pages)
        for logical in partition["exact_logical_pages"]:
            exact_map[logical] = pt.exact_physical_page_index(
                request, logical, self.exact_tail_pages, self.exact_sink_pages,
                self.exact_static_suffix_pages, self.initial_context_pages)
        base = request * self.pages_per_request
        prefill_page_gauge(key, value, kc, vc,
                           self.key_codes[layer, base:base + pages],
                           self.value_codes[layer, base:base + pages],
                           self.key_scales[layer, base:base + pages],
                           self.value_scales[layer, base:base + pages],
                           exact_map.to(key.device), self.exact_key[layer], self.exact_value[layer])


# ---------------------------------------------------------------------------
# Plan guard
# ---------------------------------------------------------------------------

class SegmentTable:
    """Device page table of one decode segment with a structural-signature
    guard (``GraphDecodeWrapper.plan``, scripts/benchmark_page_gauge_transformer.py:1517-1580).

    ``plan`` keeps the device ``last_len`` current (the kernels re-read it on
    every run, so a captured graph stays valid across the 16 steps of a page);
    it launches the fill only when the value changes, since every fill between
    two graph replays is a launch the GPU waits for.  indptr/indices are
    rewritten only when the signature changes.  The
    signature is (batch, pages per request, split, table storage, epoch): the
    work list of the split scheduler depends on page counts only, not on the
    number of tokens in the last page.  Returns True when the table changed.
    """

    def __init__(self, batch_size: int, max_pages: int, device="cuda") -> None:
        self.batch_size = batch_size
        self.indptr = torch.empty(batch_size + 1, device=device, dtype=torch.int32)
        self.indices = torch.empty(batch_size * max_pages, device=device, dtype=torch.int32)
        self.last_len = torch.full((batch_size,), PAGE, device=device, dtype=torch.int32)
        self._device_last_len = PAGE     # the value ``last_len`` holds on the device
        self.host_indptr: Optional[torch.Tensor] = None
        self.host_last_len: Optional[torch.Tensor] = None
        self.signature: Optional[tuple] = None
        self.pages_per_request = 0
        self.plan_invocations = 0
        self.plan_rebuilds = 0
        self.last_len_fills = 0

    def operation_counts(self) -> dict[str, int]:
        return {"plan_invocations": self.plan_invocations,
                "plan_rebuilds": self.plan_rebuilds,
                "last_page_len_device_fills": self.last_len_fills}

    def plan(self, physical_indices: torch.Tensor, logical_tokens: int, last_page_len: int,
             split_pages: int, page_table_epoch: Optional[int] = None) -> bool:
        self.plan_invocations += 1
        if physical_indices.dim() == 1:
            if self.batch_size != 1:
                raise ValueError("batched page indices must be [B,pages]")
            physical_indices = physical_indices.view(1, -1)
        if physical_indices.dim() != 2 or int(physical_indices.shape[0]) != self.batch_size:
            raise ValueError("physical page indices must have shape [B,pages]")
        pages = int(physical_indices.shape[1])
        if pages <= 0:
            raise ValueError("decode segment must contain at least one page")
        if not 1 <= last_page_len <= PAGE or logical_tokens != (pages - 1) * PAGE + last_page_len:
            raise ValueError("logical tokens do not match the page count and last page length")
        total = self.batch_size * pages
        if total > self.indices.numel():
            raise ValueError("decode segment exceeds the allocated page table")
        if last_page_len != self._device_last_len:
            self.last_len.fill_(last_page_len)
            self._device_last_len = last_page_len
            self.last_len_fills += 1
        self.host_last_len = torch.full((self.batch_size,), last_page_len, dtype=torch.int32)
        signature = (self.batch_size, pages, int(split_pages), physical_indices.data_ptr(),
                     page_table_epoch)
        if signature == self.signature:
            return False
        self.plan_rebuilds += 1
        self.host_indptr = torch.arange(0, total + 1, pages, dtype=torch.int32)
        self.indptr.copy_(self.host_indptr)
        self.indices[:total].view(self.batch_size, pages).copy_(physical_indices)
        self.pages_per_request = pages
        self.signature = signature
        return True

    def active_indices(self) -> torch.Tensor:
        return self.indices[:self.batch_size * self.pages_per_request]


# ---------------------------------------------------------------------------
# Decoder
# ---------------------------------------------------------------------------

class PageGaugeDecoder:
    """``TransformerDecoder`` (scripts/benchmark_page_gauge_transformer.py:1583-3275)
    for the ``page_gauge`` and ``fp16`` backends, batch ``B`` synchronised
    requests, device-dynamic positions and whole-step graphs."""

    def __init__(self, weights: DecoderWeights, cache, backend: str, max_context: int,
                 rope_cos: torch.Tensor, rope_sin: torch.Tensor, exact_tail: int = 256,
                 split_pages: int = 0, batch_size: int = 1, exact_sink_pages: int = 0,
                 workspace_bytes: int = 128 * 1024 * 1024, fused: Optional[bool] = None,
                 tail_attention: str = "segmented", fused_append: Optional[bool] = None,
                 exact_static_suffix_pages: int = 0,
                 initial_context_pages: Optional[int] = None) -> None:
        if backend not in ("page_gauge", "fp16"):
            raise ValueError(f"unknown backend {backend}")
        if tail_attention not in ("segmented", "heterogeneous"):
            raise ValueError(f"unknown exact-tail attention path {tail_attention}")
        if tail_attention == "heterogeneous" and exact_sink_pages:
            raise ValueError("exact prefix pages require the segmented flashinfer_merge path")
        layout = pt.ExactPageLayout.checked(exact_sink_pages, exact_static_suffix_pages,
                                            initial_context_pages, exact_tail // PAGE)
        if layout.suffix and tail_attention != "segmented":
            raise ValueError("an exact static suffix requires the segmented flashinfer_merge path")
        self.tail_attention = tail_attention
        if batch_size <= 0:
            raise ValueError("batch size must be positive")
        if exact_tail <= 0 or exact_tail % PAGE:
            raise ValueError("exact tail must be a positive multiple of 16 tokens")
        cfg = weights.config
        if (rope_cos.dtype != torch.float16 or rope_cos.shape != rope_sin.shape
                or rope_cos.dim() != 2 or int(rope_cos.shape[1]) != DIM
                or not rope_cos.is_contiguous() or not rope_sin.is_contiguous()
                or not rope_cos.is_cuda):
            raise ValueError("RoPE tables must be matching contiguous CUDA FP16 [positions,128]")
        self.weights = weights
        self.config = cfg
        self.backend = backend
        self.cache = cache
        self.batch_size = batch_size
        self.max_pages = math.ceil(max_context / PAGE)
        self.exact_tail_pages = exact_tail // PAGE
        self.exact_sink_pages = layout.prefix
        self.exact_static_suffix_pages = layout.suffix
        self.initial_context_pages = layout.initial
        self.exact_fixed_pages = layout.fixed           # slots that never move: S + A
        exact_slots = layout.fixed + self.exact_tail_pages
        self.split_pages = split_pages
        self.rope_cos, self.rope_sin = rope_cos, rope_sin
        device = rope_cos.device
        self.append_extension = load_append_extension()
        self.workspace = torch.empty(workspace_bytes, device=device, dtype=torch.uint8)
        self.all_pages = pt.request_major_page_table(batch_size, self.max_pages, device=device)
        if backend == "page_gauge":
            if not isinstance(cache, GaugeCache) or cache.pages_per_request != self.max_pages:
                raise ValueError("PageGauge cache must use request-major pages and per-request "
                                 "[L,B,Hkv,D] centers")
            if (cache.exact_tail_pages != self.exact_tail_pages
                    or cache.exact_sink_pages != self.exact_sink_pages
                    or cache.exact_static_suffix_pages != self.exact_static_suffix_pages
                    or cache.initial_context_pages != self.initial_context_pages):
                raise ValueError("exact cache must contain the configured fixed prefix/suffix "
                                 "pages followed by tail-ring pages")
            self.exact_ring_pages = pt.request_major_exact_page_table(
                batch_size, self.max_pages, self.exact_tail_pages, self.exact_sink_pages,
                self.exact_static_suffix_pages, self.initial_context_pages, device=device)
            self.exact_plan_pages = torch.empty(batch_size, exact_slots, device=device,
                                                dtype=torch.int32)
            # with a static suffix the INT8 pages are no longer one run of the
            # logical table: they are gathered into a table of their own
            self.old_plan_pages = (torch.empty_like(self.all_pages)
                                   if self.exact_static_suffix_pages else None)
            self.old_layout_signature: Optional[tuple] = None
            self.old_page_table_updates = 0
            if tail_attention == "heterogeneous":
                # one unified table: INT8 code pages, then the exact ring
                # (scripts/benchmark_page_gauge_transformer.py:1817-1830, :2085-2110)
                self.heterogeneous_pages = torch.empty_like(self.all_pages)
                self.old_kv_len = torch.zeros(batch_size, device=device, dtype=torch.int32)
                self.heterogeneous_layout: Optional[tuple] = None
                self.heterogeneous_page_table_updates = 0
                self.table = SegmentTable(batch_size, self.max_pages, device)
                self.decode = HeterogeneousDecodeWrapper(self.workspace)
            else:
                self.old_table = SegmentTable(batch_size, self.max_pages, device)
                self.exact_table = SegmentTable(batch_size, exact_slots, device)
                self.decode = PageGaugeSegmentedDecode(self.workspace)
        else:
            if not isinstance(cache, Fp16Cache) or cache.pages_per_request != self.max_pages:
                raise ValueError("baseline cache must use request-major [L,B*P,16,Hkv,D] storage")
            self.table = SegmentTable(batch_size, self.max_pages, device)
            self.decode = BatchDecodeWithPagedKVCacheWrapper(self.workspace, "NHD")
        self.exact_layout_signature: Optional[tuple] = None
        self.exact_page_table_updates = 0
        self.device_position = torch.zeros(1, device=device, dtype=torch.int32)
        self.rotated_query = torch.empty(batch_size, cfg.q_heads, DIM, device=device,
                                         dtype=torch.float16)
        self.attention_output = torch.empty(cfg.layers, batch_size, cfg.q_heads, DIM,
                                            device=device, dtype=torch.float16)
        self.current_pages = 0
        self.old_pages = 0
        self.exact_pages = 0
        self.tail_logical_begin = 0
        self.plan_signature_value: Optional[tuple] = None
        self.decoder_plan_calls = 0
        self.kernel_replans = 0
        # whole-step graphs, banked by plan signature
        self.graph_bank: dict[tuple, torch.cuda.CUDAGraph] = {}
        self.graph_token = torch.zeros(batch_size, device=device, dtype=torch.int64)
        self.graph_logits = torch.empty(batch_size, cfg.vocab, device=device, dtype=torch.float32)
        self.graph_next = torch.zeros(batch_size, device=device, dtype=torch.int64)
        self.graph_replays = 0
        self.eager_steps = 0
        self.graph_bank_misses = 0
        # fused projections (pg_decoder_gemv): batch <= 4, widths multiples of
        # 512, and batch * width <= 32768 unless the width is 4096 or 14336
        ok = batch_size <= 4 and all(
            w % 512 == 0 and (w in (4096, 14336) or batch_size * w <= 32768)
            for w in (cfg.hidden, cfg.intermediate))
        self.fused = ok if fused is None else fused
        if self.fused and not ok:
            raise ValueError("fused projections need batch <= 4 and widths that are multiples "
                             "of 512 (4096 / 14336, or batch * width <= 32768)")
        # the QKV projection carries the cache update (pg_decoder_qkv_rope_append;
        # the PageGauge page finalize then runs in the decode's FP16 pass)
        append_ok = self.fused and cfg.hidden == 4096
        self.fused_append = append_ok if fused_append is None else fused_append
        if self.fused_append and not append_ok:
            raise ValueError("the fused cache update needs fused projections and hidden 4096")
        self._hidden = torch.empty(batch_size, cfg.hidden, device=device, dtype=torch.float16)
        self._qkv = torch.empty(batch_size, cfg.qkv_width, device=device, dtype=torch.float16)
        self._activation = torch.empty(batch_size, cfg.intermediate, device=device,
                                       dtype=torch.float16)
        self._logits = torch.empty(batch_size, cfg.vocab, device=device, dtype=torch.float32)

    # -- plan --------------------------------------------------------------
    def plan(self, context: int) -> None:
        """Partition ``context`` tokens and (re)plan the decode work list only
        when the page structure changes (:2034-2155)."""
        self.decoder_plan_calls += 1
        pages = math.ceil(context / PAGE)
        if context <= 0 or pages > self.max_pages:
            raise ValueError("context lies outside the allocated cache capacity")
        last_len = (context - 1) % PAGE + 1
        self.current_pages = pages
        if self.backend == "fp16":
            changed = self.table.plan(self.all_pages[:, :pages], context, last_len,
                                      self.split_pages)
            if changed:
                self.decode.plan(self.table.host_indptr, self.table.active_indices(),
                                 self.table.last_len, self.config.q_heads, self.config.kv_heads,
                                 DIM, PAGE, kv_data_type=torch.float16,
                                 fixed_split_size=self.split_pages or None)
                self.kernel_replans += 1
            self.plan_signature_value = ("fp16", self.table.signature)
            return
        partition = pt.page_gauge_logical_partition(pages, self.exact_tail_pages,
                                                    self.exact_sink_pages, last_len,
                                                    self.exact_static_suffix_pages,
                                                    self.initial_context_pages)
        self.tail_logical_begin = int(partition["tail_logical_begin"])
        self.old_pages = int(partition["old_page_count"])
        self.exact_pages = int(partition["exact_page_count"])
        old_tokens = int(partition["old_token_count"])
        exact_tokens = int(partition["exact_token_count"])
        if self.tail_attention == "heterogeneous":
            layout = (self.old_pages, pages)
            if layout != self.heterogeneous_layout:
                pt.write_heterogeneous_page_table(self.heterogeneous_pages, self.all_pages,
                                                  self.exact_ring_pages, self.old_pages, pages)
                self.old_kv_len.fill_(old_tokens)
                self.heterogeneous_layout = layout
                self.heterogeneous_page_table_updates += 1
            if self.table.plan(self.heterogeneous_pages[:, :pages], context, last_len,
                               self.split_pages, page_table_epoch=self.heterogeneous_page_table_updates):
                self.decode.plan(self.table.host_indptr, self.table.active_indices(),
                                 self.table.last_len, self.config.q_heads, self.config.kv_heads,
                                 DIM, PAGE, fixed_split_size=self.split_pages or None,
                                 exact_tail_pages_hint=self.exact_pages)
                self.kernel_replans += 1
            self.plan_signature_value = ("heterogeneous", self.table.signature)
            return
        old_epoch = None
        if self.old_plan_pages is not None:
            # for a fixed prefix, suffix and ring the INT8 set grows one page
            # at a time, so its size names it
            layout = (self.old_pages,)
            if layout != self.old_layout_signature:
                old_indices = pt.write_page_gauge_old_page_table(
                    self.old_plan_pages, self.all_pages, partition["old_logical_pages"])
                self.old_layout_signature = layout
                self.old_page_table_updates += 1
            else:
                old_indices = self.old_plan_pages[:, :self.old_pages]
            old_epoch = self.old_page_table_updates
        else:
            old_begin = partition["old_logical_pages"][0]
            old_indices = self.all_pages[:, old_begin:old_begin + self.old_pages]
        changed = self.old_table.plan(old_indices, old_tokens, PAGE, self.split_pages,
                                      page_table_epoch=old_epoch)
        epoch = None
        if self.exact_fixed_pages:
            layout = (self.tail_logical_begin, pages, self.exact_pages)
            if layout != self.exact_layout_signature:
                exact_indices = pt.write_exact_prefix_tail_page_table(
                    self.exact_plan_pages, self.exact_ring_pages, self.tail_logical_begin, pages,
                    self.exact_sink_pages, self.exact_static_suffix_pages,
                    self.initial_context_pages)
                self.exact_layout_signature = layout
                self.exact_page_table_updates += 1
            else:
                exact_indices = self.exact_plan_pages[:, :self.exact_pages]
            epoch = pages
        else:
            exact_indices = self.exact_ring_pages[:, self.tail_logical_begin:pages]
        changed |= self.exact_table.plan(exact_indices, exact_tokens, last_len, self.split_pages,
                                         page_table_epoch=epoch)
        if changed:
            self.decode.plan(self.old_table.host_indptr, self.old_table.active_indices(),
                             self.old_table.last_len, self.exact_table.host_indptr,
                             self.exact_table.active_indices(), self.exact_table.last_len,
                             self.config.q_heads, self.config.kv_heads, DIM, PAGE,
                             fixed_split_size=self.split_pages or None)
            self.kernel_replans += 1
        self.plan_signature_value = ("page_gauge", self.old_table.signature,
                                     self.exact_table.signature)

    def plan_signature(self) -> Optional[tuple]:
        return self.plan_signature_value

    # -- one layer -----------------------------------------------------------
    def _append(self, layer: int, query, key, value) -> None:
        if self.backend == "fp16":
            self.append_extension.rope_append_fp16_dynamic(
                query, key, value, self.rope_cos, self.rope_sin, self.device_position,
                self.rotated_query, self.cache.key[layer], self.cache.value[layer])
            return
        c = self.cache
        self.append_extension.rope_append_page_gauge_dynamic(
            query, key, value, self.rope_cos, self.rope_sin, self.device_position,
            c.key_center[layer], c.value_center[layer], self.rotated_query, c.exact_key[layer],
            c.exact_value[layer], c.key_codes[layer], c.value_codes[layer], c.key_scales[layer],
            c.value_scales[layer], self.exact_fixed_pages)

    def _qkv_append(self, layer: int) -> None:
        """QKV projection + RoPE + cache append in one launch."""
        cfg = self.config
        w = self.weights.layers[layer]
        c = self.cache
        common = dict(norm_weight=w["input_norm"], eps=cfg.rms_eps, query_heads=cfg.q_heads,
                      kv_heads=cfg.kv_heads, cos=self.rope_cos, sin=self.rope_sin,
                      positions=self.device_position, rotated_query=self.rotated_query)
        if self.backend == "fp16":
            qkv_rope_append(w["qkv"], self._hidden, key_pages=c.key[layer],
                            value_pages=c.value[layer], key_center=None, value_center=None,
                            pages_per_request=c.pages_per_request, sink_pages=0,
                            capacity_tokens=c.pages_per_request * PAGE, **common)
            return
        qkv_rope_append(w["qkv"], self._hidden, key_pages=c.exact_key[layer],
                        value_pages=c.exact_value[layer], key_center=c.key_center[layer],
                        value_center=c.value_center[layer],
                        pages_per_request=c.exact_storage_pages_per_request,
                        sink_pages=self.exact_fixed_pages,
                        capacity_tokens=c.pages_per_request * PAGE, **common)

    def attention(self, layer: int) -> torch.Tensor:
        out = self.attention_output[layer]
        if self.backend == "fp16":
            return self.decode.run(self.rotated_query, (self.cache.key[layer],
                                                        self.cache.value[layer]), out=out)
        c = self.cache
        value_center = c.value_center[layer]
        # with the fused cache update, the decode finalizes a completed page
        finalize = (self.device_position, c.pages_per_request) if self.fused_append else None
        if self.tail_attention == "heterogeneous":
            return self.decode.run(self.rotated_query, (c.key_codes[layer], c.value_codes[layer]),
                                   c.key_scales[layer], c.value_scales[layer], c.exact_key[layer],
                                   c.exact_value[layer], self.old_kv_len, value_center, out=out,
                                   finalize=finalize)
        return self.decode.run(self.rotated_query, (c.key_codes[layer], c.value_codes[layer]),
                               c.key_scales[layer], c.value_scales[layer],
                               (c.exact_key[layer], c.exact_value[layer]),
                               value_center=value_center, out=out, finalize=finalize)

    def _layer_fused(self, layer: int) -> None:
        """One layer on ``self._hidden`` in place: 4 projection launches (the
        QKV one carrying the cache update) + K1, or with ``fused_append`` off,
        4 projections + K2 + K1."""
        cfg = self.config
        w = self.weights.layers[layer]
        b = self.batch_size
        qw, kw = cfg.q_heads * DIM, cfg.kv_heads * DIM
        if self.fused_append:
            self._qkv_append(layer)
        else:
            qkv = projection(w["qkv"], self._hidden, self._qkv, norm_weight=w["input_norm"],
                             eps=cfg.rms_eps)
            self._append(layer, qkv[:, :qw].view(b, cfg.q_heads, DIM),
                         qkv[:, qw:qw + kw].view(b, cfg.kv_heads, DIM),
                         qkv[:, qw + kw:].view(b, cfg.kv_heads, DIM))
        attended = self.attention(layer)
        projection(w["o"], attended.view(b, qw), self._hidden, residual=self._hidden)
        projection(w["gate_up"], self._hidden, self._activation, norm_weight=w["post_norm"],
                   eps=cfg.rms_eps, swiglu=True)
        projection(w["down"], self._activation, self._hidden, residual=self._hidden)

    def _layer(self, layer: int, hidden: torch.Tensor) -> torch.Tensor:
        cfg = self.config
        w = self.weights.layers[layer]
        b = self.batch_size
        x = rms_norm(hidden, w["input_norm"], cfg.rms_eps)
        qkv = F.linear(x, w["qkv"])
        qw, kw = cfg.q_heads * DIM, cfg.kv_heads * DIM
        query = qkv[:, :qw].view(b, cfg.q_heads, DIM)
        key = qkv[:, qw:qw + kw].view(b, cfg.kv_heads, DIM)
        value = qkv[:, qw + kw:].view(b, cfg.kv_heads, DIM)
        self._append(layer, query, key, value)
        attended = self.attention(layer)
        hidden = hidden + F.linear(attended.reshape(b, qw), w["o"])
        x = rms_norm(hidden, w["post_norm"], cfg.rms_eps)
        gate, up = F.linear(x, w["gate_up"]).split(cfg.intermediate, dim=-1)
        return hidden + F.linear(F.silu(gate) * up, w["down"])

    def _body(self, token: torch.Tensor) -> torch.Tensor:
        if self.fused:
            torch.index_select(self.weights.embed, 0, token.reshape(self.batch_size),
                               out=self._hidden)
            for layer in range(self.config.layers):
                self._layer_fused(layer)
            return projection(self.weights.lm_head, self._hidden, self._logits,
                              norm_weight=self.weights.norm, eps=self.config.rms_eps)
        hidden = F.embedding(token.reshape(self.batch_size), self.weights.embed)
        for layer in range(self.config.layers):
            hidden = self._layer(layer, hidden)
        normalized = rms_norm(hidden, self.weights.norm, self.config.rms_eps)
        return F.linear(normalized, self.weights.lm_head).float()

    # -- steps -----------------------------------------------------------------
    def _prepare(self, token: torch.Tensor, position: int) -> None:
        if token.numel() != self.batch_size:
            raise ValueError(f"expected {self.batch_size} synchronized tokens, got {token.numel()}")
        if not 0 <= position < int(self.rope_cos.shape[0]):
            raise ValueError("decode position lies outside the allocated RoPE table")
        self.plan(position + 1)
        self.device_position.fill_(position)

    @torch.inference_mode()
    def step(self, token: torch.Tensor, position: int) -> torch.Tensor:
        """One decode step for synchronized requests at ``position``; returns
        float32 logits [B, vocab].  Replays the banked graph of the current
        plan signature when one was captured, else runs eagerly."""
        self._prepare(token, position)
        graph = self.graph_bank.get(self.plan_signature())
        if graph is None:
            if self.graph_bank:
                self.graph_bank_misses += 1
            self.eager_steps += 1
            return self._body(token)
        if token.data_ptr() != self.graph_token.data_ptr():
            self.graph_token.copy_(token.reshape(self.batch_size))
        graph.replay()
        self.graph_replays += 1
        return self.graph_logits

    @torch.inference_mode()
    def capture(self, position: int, warmups: int = 1) -> None:
        """Capture the whole step at ``position``'s plan signature.  The step
        is executed ``warmups`` times eagerly first; callers must restore the
        cache slot of ``position`` afterwards if its contents matter (the
        replay at that position rewrites it identically)."""
        token = self.graph_token
        self._prepare(token, position)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(warmups):
                self._body(token)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = self._body(token)
            self.graph_logits.copy_(logits)
            if self.fused:
                argmax_rows(self.graph_logits, self.graph_next)
            else:
                torch.argmax(self.graph_logits, dim=-1, out=self.graph_next)
        self.graph_bank[self.plan_signature()] = graph

    def drop_graphs(self) -> None:
        self.graph_bank.clear()

    @torch.inference_mode()
    def generate(self, first_token: torch.Tensor, start_position: int, steps: int,
                 use_graphs: bool = True) -> tuple[torch.Tensor, list[torch.Tensor]]:
        """Greedy decode of ``steps`` tokens; returns (tokens [steps, B],
        per-step float32 logits).  With graphs the argmax is part of the
        captured step and the next token never leaves the device."""
        tokens, logits_seq = [], []
        token = first_token.reshape(self.batch_size).to(torch.int64)
        for i in range(steps):
            position = start_position + i
            if use_graphs and self.plan_signature_after(position) not in self.graph_bank:
                self.capture(position)
            logits = self.step(token, position)
            if use_graphs and self.plan_signature() in self.graph_bank:
                token = self.graph_next.clone()
            elif self.fused:
                token = argmax_rows(logits, torch.empty(self.batch_size, dtype=torch.int64,
                                                        device=logits.device))
            else:
                token = logits.argmax(dim=-1)
            tokens.append(token)
            logits_seq.append(logits.clone())
        return torch.stack(tokens), logits_seq

    def plan_signature_after(self, position: int) -> Optional[tuple]:
        """Signature ``plan(position + 1)`` would produce (plans if needed)."""
        self.plan(position + 1)
        return self.plan_signature()

    def counts(self) -> dict[str, Any]:
        out = {"decoder_plan_calls": self.decoder_plan_calls, "kernel_replans": self.kernel_replans,
               "graph_replays": self.graph_replays, "eager_steps": self.eager_steps,
               "graph_bank_misses": self.graph_bank_misses,
               "exact_page_table_updates": self.exact_page_table_updates}
        if self.backend == "fp16" or self.tail_attention == "heterogeneous":
            out["table"] = self.table.operation_counts()
        else:
            out["old_table"] = self.old_table.operation_counts()
            out["exact_table"] = self.exact_table.operation_counts()
        return out


def build_decoders(weights: DecoderWeights, prompt: torch.Tensor, decode_steps: int,
                   exact_tail: int = 256, backends=("page_gauge", "fp16"), split_pages: int = 0,
                   exact_sink_pages: int = 0, exact_static_suffix_pages: int = 0):
    """Prefill ``prompt`` [T] or [B, T] (T a multiple of 16; every request the
    same length, as the decoder steps requests in lockstep) once per request,
    populate one cache per backend from the same rotated K/V, and return
    ``(first_tokens [B], prefill_logits [B,V], {backend: decoder})``.  A
    static suffix keeps the last ``exact_static_suffix_pages`` pages of the
    prompt exact (the initial context is the prompt)."""
    cfg = weights.config
    prompts = prompt.reshape(1, -1) if prompt.dim() == 1 else prompt
    batch, count = int(prompts.shape[0]), int(prompts.shape[1])
    if count % PAGE or count <= exact_tail + PAGE * exact_sink_pages:
        raise SystemExit("context and exact tail must be page aligned; context must be larger")
    max_context = count + decode_steps + 1
    pages = math.ceil(max_context / PAGE)
    device = weights.embed.device
    cos, sin = rope_tables(max_context, cfg.rope_theta)
    cos, sin = cos.to(device), sin.to(device)
    caches = {}
    initial = count // PAGE if exact_static_suffix_pages else None
    if "page_gauge" in backends:
        caches["page_gauge"] = GaugeCache(cfg, batch, pages, exact_tail // PAGE, exact_sink_pages,
                                          device, exact_static_suffix_pages, initial)
    if "fp16" in backends:
        caches["fp16"] = Fp16Cache(cfg, batch, pages, device)

    logits = []
    for request in range(batch):
        def on_layer(layer, key, value, request=request):
            for cache in caches.values():
                cache.populate(layer, request, key, value)

        logits.append(prefill(weights, prompts[request].to(device), cos, sin, on_layer))
    logits = torch.cat(logits)
    first = logits.argmax(dim=-1)
    decoders = {name: PageGaugeDecoder(
                    weights, cache, name, max_context, cos, sin, exact_tail, split_pages, batch,
                    exact_sink_pages if name == "page_gauge" else 0,
                    exact_static_suffix_pages=exact_static_suffix_pages if name == "page_gauge" else 0,
                    initial_context_pages=initial if name == "page_gauge" else None)
                for name, cache in caches.items()}
    return first, logits, decoders
