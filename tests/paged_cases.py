"""Seeded inputs of the paged fp8 / bf16 tests and benchmark: bf16 q/K/V from N(0, 1), per-head scales, a shuffled
block table, and the oracle's view of the same cache (codes decoded with the reference's fp8_decode)."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle import paged as opaged
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits

FMT_NAME = {torch.float8_e4m3fn: "e4m3", torch.float8_e5m2: "e5m2"}


def bf16_normal(shape, generator: torch.Generator, scale: float = 1.0) -> torch.Tensor:
    return (torch.randn(*shape, generator=generator) * scale).to(torch.bfloat16)


def to_numpy_f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@dataclass
class PagedCase:
    q: torch.Tensor  # [B, Q, Hq, D] bf16 (CPU)
    k: torch.Tensor  # [B, Hkv, S, D] bf16 (CPU), full precision
    v: torch.Tensor
    lens: list[int]
    table: np.ndarray
    pages: int
    dtype: torch.dtype
    k_scale: np.ndarray | None
    v_scale: np.ndarray | None
    k_codes: np.ndarray  # cache elements [B, Hkv, S, D]: fp8 bytes or bf16 bit patterns
    v_codes: np.ndarray

    def decoded(self, out: str = "f32") -> tuple[np.ndarray, np.ndarray]:
        """K/V as the fused kernel's definition sees them, float32 [B, Hkv, S, D]: ``fp8_decode`` (fp8.py:89-92)
        with ``out`` float32, i.e. every byte's exact value times its head's scale in fp32 (the reference's fused fp8
        kernel reads the bytes exactly and rounds nothing; the per-head scale multiplies in fp32). ``out="bf16"``
        gives the non-fused cache's values, rounded to the model dtype."""
        if self.dtype == torch.bfloat16:
            return bf16_bits_to_f32(self.k_codes), bf16_bits_to_f32(self.v_codes)
        fmt = FMT_NAME[self.dtype]
        ks = self.k_scale.reshape(1, -1, 1, 1)
        vs = self.v_scale.reshape(1, -1, 1, 1)
        return ofp8.fp8_decode(self.k_codes, fmt, ks, out), ofp8.fp8_decode(self.v_codes, fmt, vs, out)

    def device_cache(self, device: str = "cuda", poison: bool = False):
        """The paged cache on ``device``. With ``poison`` every slot the rows do not hold (the tail of each row's
        last page and every unused page) holds NaN codes instead of zeros, as never-written cache memory may."""
        from economize_amd.paged import PagedKVCache

        element = 2 if self.dtype == torch.bfloat16 else 1
        kc, vc = opaged.scatter_kv(self.k_codes, self.v_codes, self.lens, self.table, self.pages, 16, element)
        if poison:
            held_k, held_v = opaged.scatter_kv(np.ones_like(self.k_codes), np.ones_like(self.v_codes), self.lens,
                                               self.table, self.pages, 16, element)
            nan = np.array(0xFFFF if element == 2 else 0xFF, dtype=kc.dtype)
            kc = np.where(held_k != 0, kc, nan)
            vc = np.where(held_v != 0, vc, nan)
        raw = torch.int16 if element == 2 else torch.uint8
        keys = torch.from_numpy(kc.view(np.int16) if element == 2 else kc).to(raw).view(self.dtype).to(device)
        values = torch.from_numpy(vc.view(np.int16) if element == 2 else vc).to(raw).view(self.dtype).to(device)
        ks = None if self.k_scale is None else torch.from_numpy(self.k_scale).to(device)
        vs = None if self.v_scale is None else torch.from_numpy(self.v_scale).to(device)
        return PagedKVCache(keys.contiguous(), values.contiguous(), ks, vs)


def make_case(batch: int, queries: int, q_heads: int, kv_heads: int, head_dim: int, lens, dtype: torch.dtype,
              seed: int = 0, scaled: bool = True) -> PagedCase:
    gen = torch.Generator().manual_seed(seed)
    smax = max(max(lens), 1)
    q = bf16_normal((batch, queries, q_heads, head_dim), gen)
    k = bf16_normal((batch, kv_heads, smax, head_dim), gen)
    v = bf16_normal((batch, kv_heads, smax, head_dim), gen)
    table, pages = opaged.shuffled_block_table(lens, 16, seed=seed + 1)
    kf, vf = to_numpy_f32(k), to_numpy_f32(v)
    mask = np.zeros((batch, 1, smax, 1), bool)
    for b, n in enumerate(lens):
        mask[b, :, :n] = True
    if dtype == torch.bfloat16:
        return PagedCase(q, k, v, list(lens), table, pages, dtype, None, None, f32_to_bf16_bits(kf),
                         f32_to_bf16_bits(vf))
    fmt = FMT_NAME[dtype]
    if scaled:
        # per-head absmax over the tokens each row holds (the calibration sees the cache's entries)
        ks = ofp8.head_scales(np.where(mask, kf, 0), fmt)
        vs = ofp8.head_scales(np.where(mask, vf, 0), fmt)
    else:
        ks = np.ones(kv_heads, np.float32)
        vs = np.ones(kv_heads, np.float32)
    kc = ofp8.fp8_encode(kf, fmt, ks.reshape(1, -1, 1, 1))
    vc = ofp8.fp8_encode(vf, fmt, vs.reshape(1, -1, 1, 1))
    return PagedCase(q, k, v, list(lens), table, pages, dtype, ks, vs, kc, vc)


def oracle_output(case: PagedCase, scale: float | None = None, softcap=None, sinks=None) -> np.ndarray:
    """``[B, Q, Hq, D]`` float32: the fp32 definition over the decoded cache with causal, per-length masks."""
    from oracle.attention import reference_attention

    kd, vd = case.decoded()
    q = to_numpy_f32(case.q).transpose(0, 2, 1, 3)  # [B, Hq, Q, D]
    batch, hq, nq, d = q.shape
    smax = kd.shape[2]
    mask = np.zeros((batch, 1, nq, smax), bool)
    for b, n in enumerate(case.lens):
        for qi in range(nq):
            mask[b, 0, qi, : max(0, n - nq + qi + 1)] = True
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    return reference_attention(q, kd, vd, mask, scale, softcap=softcap, sinks=sinks)
