"""Synthetic decode workloads of the benchmark configurations.

Seeded inputs are generated on the CPU with ``torch.Generator`` (so the same
seed gives the same tensors on any machine), then copied to the device.  Each
request's channel centers are the exact token mean of its whole context
(``token_major_centers``), and its INT8 history pages are quantised on the GPU
as the reference's K1 driver builds its caches (``quantize_page_gauge``,
scripts/benchmark_flashinfer_page_affine_int8.py:256-278 and :489-494:
float32-centered values, round-half-even codes), or with
``quantizer="completed_pages"`` by the prefill bulk quantizer
(``pg_quantize_completed_kv_pages``: sign-symmetric rounding); the newest
``tail_tokens`` tokens are kept as a centered FP16 ring.  Physical page ids are
a seeded random permutation of a shared pool.

Configurations (shapes of the reference's Mistral-7B layer: 32 query heads,
8 KV heads, head_dim 128, 16-token pages):
  * ``b1_49k``:  one request, 49152 tokens = 3056 INT8 pages + 16 FP16 pages,
    K/V ~ N(0,1) with x8 on 4 of 128 channels (separately for K and V);
  * ``single_4k``: one request, 4096 tokens (3840 INT8 + 256 FP16);
  * ``b8_ragged``: 8 requests with lengths U[4096, 32768] (multiples of 16);
  * ``serving_b256``: 256 requests of 16-240 INT8 pages behind full rings;
  * arbitrary lengths through ``build_decode_workload``.
"""

from __future__ import annotations

import random

from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from .update import quantize_completed_kv_pages, quantize_page_gauge, token_major_centers

HQ = 32
HKV = 8
DIM = 128
PAGE = 16
TAIL_TOKENS = 256
VALIDATION_SEEDS = (20260840, 20260841, 20260842, 20260843, 20260844)
PILOT_SEED = 20260814


@dataclass
class DecodeWorkload:
    """Device tensors of one paged-decode problem (INT8 history + FP16 tail)."""

    lengths: list[int]
    query: torch.Tensor             # [B, 32, 128] fp16
    k_codes: torch.Tensor           # [N, 16, 8, 128] int8 (shared pool)
    v_codes: torch.Tensor
    k_scale: torch.Tensor           # [N, 8] fp16
    v_scale: torch.Tensor
    old_indptr: torch.Tensor        # [B+1] int32
    old_indices: torch.Tensor       # int32
    old_last_page_len: torch.Tensor  # [B] int32 (16: history pages are whole)
    tail_k: torch.Tensor            # [E, 16, 8, 128] fp16 centered ring pool
    tail_v: torch.Tensor
    tail_indptr: torch.Tensor
    tail_indices: torch.Tensor
    tail_last_page_len: torch.Tensor
    key_center: torch.Tensor        # [B, 8, 128] fp16
    value_center: torch.Tensor
    sm_scale: float = DIM ** -0.5
    fp16_k: Optional[torch.Tensor] = None   # centered FP16 copy of every page (same-way kernel)
    fp16_v: Optional[torch.Tensor] = None
    fp16_indptr: Optional[torch.Tensor] = None
    fp16_indices: Optional[torch.Tensor] = None
    fp16_last_page_len: Optional[torch.Tensor] = None
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return len(self.lengths)

    def algorithmic_bytes(self) -> int:
        """Compulsory HBM bytes of one INT8+tail decode call.

        INT8 codes (K+V) + page scales (K+V) + FP16 tail (K+V) + page tables
        + q + out + lse + value center.
        """
        old_pages = int(self.old_indices.numel())
        tail_pages = int(self.tail_indices.numel())
        per_old = 2 * PAGE * HKV * DIM + 2 * HKV * 2       # codes + scales
        per_tail = 2 * PAGE * HKV * DIM * 2
        tables = 4 * (old_pages + tail_pages + 2 * (self.batch + 1) + 2 * self.batch)
        qo = self.batch * HQ * DIM * 2 * 2 + self.batch * HQ * 4
        center = self.batch * HKV * DIM * 2
        return old_pages * per_old + tail_pages * per_tail + tables + qo + center

    def fp16_algorithmic_bytes(self) -> int:
        pages = int(self.fp16_indices.numel()) if self.fp16_indices is not None else 0
        tables = 4 * (pages + 2 * self.batch + 1)
        qo = self.batch * HQ * DIM * 2 * 2 + self.batch * HQ * 4
        return pages * 2 * PAGE * HKV * DIM * 2 + tables + qo


def _outlier_kv(generator: torch.Generator, tokens: int, outlier_channels: int,
                outlier_gain: float) -> torch.Tensor:
    values = torch.randn(tokens, HKV, DIM, generator=generator, dtype=torch.float32)
    if outlier_channels:
        channels = torch.randperm(DIM, generator=generator)[:outlier_channels]
        values[:, :, channels] *= outlier_gain
    return values.to(torch.float16)


def build_decode_workload(lengths: Sequence[int], seed: int, device="cuda",
                          tail_tokens: int = TAIL_TOKENS, outlier_channels: int = 4,
                          outlier_gain: float = 8.0, shuffle_pages: bool = True,
                          with_fp16_copy: bool = False, query_scale: float = 1.0,
                          quantizer: str = "page_gauge") -> DecodeWorkload:
    """Build a seeded INT8-history + FP16-tail workload for ``lengths``.

    Each length must be a positive multiple of 16 and larger than
    ``tail_tokens``; the last ``tail_tokens`` tokens form the FP16 ring.
    """
    lengths = [int(n) for n in lengths]
    if any(n % PAGE or n <= tail_tokens for n in lengths):
        raise ValueError("lengths must be multiples of 16 longer than the tail")
    if tail_tokens % PAGE:
        raise ValueError("tail must be whole pages")
    if quantizer not in ("page_gauge", "completed_pages"):
        raise ValueError("quantizer must be 'page_gauge' or 'completed_pages'")
    generator = torch.Generator().manual_seed(seed)
    batch = len(lengths)
    query = (torch.randn(batch, HQ, DIM, generator=generator) * query_scale).to(torch.float16)
    tail_pages = tail_tokens // PAGE
    old_counts = [n // PAGE - tail_pages for n in lengths]
    total_old = sum(old_counts)
    total_tail = tail_pages * batch
    old_perm = torch.randperm(total_old, generator=generator) if shuffle_pages else torch.arange(total_old)
    tail_perm = torch.randperm(total_tail, generator=generator) if shuffle_pages else torch.arange(total_tail)

    k_codes = torch.empty(total_old, PAGE, HKV, DIM, dtype=torch.int8, device=device)
    v_codes = torch.empty_like(k_codes)
    k_scale = torch.empty(total_old, HKV, dtype=torch.float16, device=device)
    v_scale = torch.empty_like(k_scale)
    tail_k = torch.empty(total_tail, PAGE, HKV, DIM, dtype=torch.float16, device=device)
    tail_v = torch.empty_like(tail_k)
    key_centers, value_centers = [], []
    old_indices, tail_indices = [], []
    fp16_k = fp16_v = None
    fp16_indices = []
    fp16_perm = None
    if with_fp16_copy:
        fp16_k = torch.empty(total_old + total_tail, PAGE, HKV, DIM, dtype=torch.float16, device=device)
        fp16_v = torch.empty_like(fp16_k)
        fp16_perm = (torch.randperm(total_old + total_tail, generator=generator) if shuffle_pages
                     else torch.arange(total_old + total_tail))
    fp16_cursor = 0
    old_cursor = tail_cursor = 0
    for request, length in enumerate(lengths):
        keys = _outlier_kv(generator, length, outlier_channels, outlier_gain)
        values = _outlier_kv(generator, length, outlier_channels, outlier_gain)
        n_old = old_counts[request]
        ids_old = old_perm[old_cursor:old_cursor + n_old]
        ids_tail = tail_perm[tail_cursor:tail_cursor + tail_pages]
        old_cursor += n_old
        tail_cursor += tail_pages
        old_indices.append(ids_old)
        tail_indices.append(ids_tail)
        dev_k = keys.reshape(-1, PAGE, HKV, DIM).to(device)
        dev_v = values.reshape(-1, PAGE, HKV, DIM).to(device)
        # per-(request, kv head) channel centers: exact mean of the whole context
        dkc, dvc = token_major_centers(dev_k.view(-1, HKV, DIM), dev_v.view(-1, HKV, DIM))
        key_centers.append(dkc)
        value_centers.append(dvc)
        # history: quantised into the shuffled pool
        old_k = dev_k[:n_old].contiguous()
        old_v = dev_v[:n_old].contiguous()
        if quantizer == "page_gauge":
            ck, _, sk, _, _ = quantize_page_gauge(old_k, dkc)
            cv, _, sv, _, _ = quantize_page_gauge(old_v, dvc)
        else:
            ck = torch.empty(n_old, PAGE, HKV, DIM, dtype=torch.int8, device=device)
            cv = torch.empty_like(ck)
            sk = torch.empty(n_old, HKV, dtype=torch.float16, device=device)
            sv = torch.empty_like(sk)
            quantize_completed_kv_pages(old_k, old_v, dkc, dvc, ck, cv, sk, sv)
        dev_ids = ids_old.to(device)
        k_codes[dev_ids] = ck
        v_codes[dev_ids] = cv
        k_scale[dev_ids] = sk
        v_scale[dev_ids] = sv
        # tail: centered FP16 ring (fp16(f32(x) - f32(c)))
        ring_k = (dev_k[n_old:].float() - dkc.float()).to(torch.float16)
        ring_v = (dev_v[n_old:].float() - dvc.float()).to(torch.float16)
        dev_tail = ids_tail.to(device)
        tail_k[dev_tail] = ring_k
        tail_v[dev_tail] = ring_v
        if with_fp16_copy:
            full_ids = fp16_perm[fp16_cursor:fp16_cursor + n_old + tail_pages]
            fp16_cursor += n_old + tail_pages
            fp16_indices.append(full_ids)
            fp16_k[full_ids.to(device)] = (dev_k.float() - dkc.float()).to(torch.float16)
            fp16_v[full_ids.to(device)] = (dev_v.float() - dvc.float()).to(torch.float16)

    def indptr(counts):
        out = [0]
        for c in counts:
            out.append(out[-1] + c)
        return torch.tensor(out, dtype=torch.int32, device=device)

    workload = DecodeWorkload(
        lengths=lengths,
        query=query.to(device),
        k_codes=k_codes, v_codes=v_codes, k_scale=k_scale, v_scale=v_scale,
        old_indptr=indptr(old_counts),
        old_indices=torch.cat(old_indices).to(torch.int32).to(device),
        old_last_page_len=torch.full((batch,), PAGE, dtype=torch.int32, device=device),
        tail_k=tail_k, tail_v=tail_v,
        tail_indptr=indptr([tail_pages] * batch),
        tail_indices=torch.cat(tail_indices).to(torch.int32).to(device),
        tail_last_page_len=torch.full((batch,), PAGE, dtype=torch.int32, device=device),
        key_center=torch.stack(key_centers).to(device),
        value_center=torch.stack(value_centers).to(device),
        meta={"seed": seed, "outlier_channels": outlier_channels, "outlier_gain": outlier_gain,
              "tail_tokens": tail_tokens, "shuffled": shuffle_pages, "quantizer": quantizer},
    )
    if with_fp16_copy:
        workload.fp16_k = fp16_k
        workload.fp16_v = fp16_v
        workload.fp16_indptr = indptr([n // PAGE for n in lengths])
        workload.fp16_indices = torch.cat(fp16_indices).to(torch.int32).to(device)
        workload.fp16_last_page_len = torch.full((batch,), PAGE, dtype=torch.int32, device=device)
    return workload


def b1_49k(seed: int = VALIDATION_SEEDS[0], device="cuda", **kw) -> DecodeWorkload:
    return build_decode_workload([49152], seed, device=device, **kw)


def single_4k(seed: int = VALIDATION_SEEDS[0], device="cuda", **kw) -> DecodeWorkload:
    return build_decode_workload([4096], seed, device=device, **kw)


SERVING_SEED = 20261210


def serving_lengths(seed: int = SERVING_SEED, batch: int = 256) -> list[int]:
    """A serving-sized decode batch: ``batch`` requests of 16-240 INT8 pages
    (uniform, seeded) behind full 16-page FP16 rings."""
    rng = random.Random(seed)
    return [PAGE * (TAIL_TOKENS // PAGE + rng.randint(16, 240)) for _ in range(batch)]


def serving_b256(seed: int = SERVING_SEED, device="cuda", **kw) -> DecodeWorkload:
    return build_decode_workload(serving_lengths(seed), seed, device=device, **kw)


def ragged_lengths(seed: int, batch: int = 8, low: int = 4096, high: int = 32768) -> list[int]:
    generator = torch.Generator().manual_seed(seed)
    raw = torch.randint(low, high + 1, (batch,), generator=generator)
    return [max(low, int(n) // PAGE * PAGE) for n in raw]


def b8_ragged(seed: int = VALIDATION_SEEDS[0], device="cuda", **kw) -> DecodeWorkload:
    return build_decode_workload(ragged_lengths(seed), seed, device=device, **kw)
