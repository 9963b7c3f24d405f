"""KIVI 2/4-bit KV cache on the GPU: paged quantize-and-append, the residual ring and fused decode attention.

Mirrors the reference's KIVI path (Liu et al., ICML 2024):

* :class:`PagedKIVICache` holds one layer: the quantized tokens in 32-token pages (one block per page and KV head,
  see ``include/economize_amd.h``) and the most recent tokens in bf16 rings, like the reference's fused cache
  (techniques/kv_kivi_fused/fused.py:52-175) with its ring (``KIVIPacked.key_ring``, attention/kivi.py:100-108).
* :func:`kivi_append` writes new tokens into the rings; :func:`kivi_commit` runs the reference's schedule
  (techniques/kv_quant/kivi.py:230-243) on the device and quantizes what it makes due from the rings
  (``quantize``, kivi.py:121-140); :func:`kivi_quantize` quantizes a range from any source (a prompt).
* :func:`kivi_decode_attention` is ``kivi_decode_attention`` (attention/kivi.py:199-309) over the pages and rings.

Every function runs on the HIP kernels of ``libeconomize_amd.so``; there is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import _lib
from .errors import ConfigError
from .paged import cached_workspace, counter_bytes, packed_mask

__all__ = ["KIVI_PAGE", "PagedKIVICache", "kivi_append", "kivi_commit", "kivi_decode_attention", "kivi_fake_quantize",
           "kivi_gather",
           "kivi_quantize"]

#: Tokens per KIVI page.
KIVI_PAGE = 32


@dataclass
class PagedKIVICache:
    """One layer's KIVI cache.

    Attributes:
        blocks: uint8 ``[pages, Hkv, block bytes]``.
        k_ring: bf16 ``[B, Hkv, W, D]`` recent keys, token ``t`` at slot ``t % W``.
        v_ring: bf16 ``[B, Hkv, D, W]`` recent values.
        keys_quantized: int32 ``[B]`` keys below are codes.
        values_quantized: int32 ``[B]`` values below are codes.
        bits: Bits per code (2 or 4).
        group: Key tokens / value channels per scale (32).
        residual: Residual length ``R`` of the schedule (a multiple of ``group``).
        overflow: int32 ``[1]``, nonzero once a scale or zero point was beyond fp16.
    """

    blocks: torch.Tensor
    k_ring: torch.Tensor
    v_ring: torch.Tensor
    keys_quantized: torch.Tensor
    values_quantized: torch.Tensor
    bits: int
    group: int = 32
    residual: int = 128
    overflow: torch.Tensor = field(default=None)  # type: ignore[assignment]

    @classmethod
    def empty(cls, pages: int, batch: int, kv_heads: int, head_dim: int, bits: int, device: torch.device | str,
              group: int = 32, residual: int = 128, headroom: int = 256) -> PagedKIVICache:
        """A cache of ``pages`` pages and rings of ``residual + headroom`` slots (the reference's ``headroom``,
        techniques/kv_kivi_fused/fused.py:30-51); pages and rings start zeroed."""
        size = int(_lib.lib().eco_kivi_block_bytes(head_dim, bits, group))
        if size == 0:
            raise ConfigError(f"no KIVI page layout for head dim {head_dim}, {bits} bits, group {group}")
        ring = residual + headroom
        if residual % group or ring % KIVI_PAGE:
            raise ConfigError(f"residual {residual} and headroom {headroom} must keep the ring a multiple of "
                              f"{KIVI_PAGE} and the residual a multiple of the group {group}")
        return cls(
            torch.zeros(pages, kv_heads, size, dtype=torch.uint8, device=device),
            torch.zeros(batch, kv_heads, ring, head_dim, dtype=torch.bfloat16, device=device),
            torch.zeros(batch, kv_heads, head_dim, ring, dtype=torch.bfloat16, device=device),
            torch.zeros(batch, dtype=torch.int32, device=device),
            torch.zeros(batch, dtype=torch.int32, device=device),
            bits, group, residual, torch.zeros(1, dtype=torch.int32, device=device),
        )

    @property
    def num_pages(self) -> int:
        return self.blocks.shape[0]

    @property
    def kv_heads(self) -> int:
        return self.blocks.shape[1]

    @property
    def head_dim(self) -> int:
        return self.k_ring.shape[3]

    @property
    def batch(self) -> int:
        return self.k_ring.shape[0]

    @property
    def ring(self) -> int:
        return self.k_ring.shape[2]

    def check(self) -> None:
        size = int(_lib.lib().eco_kivi_block_bytes(self.head_dim, self.bits, self.group))
        if size == 0 or self.blocks.dtype != torch.uint8 or self.blocks.shape[2] != size:
            raise ConfigError(f"KIVI blocks {tuple(self.blocks.shape)} do not match head dim {self.head_dim}, "
                              f"{self.bits} bits")
        b, h, w, d = self.k_ring.shape
        if self.v_ring.shape != (b, h, d, w) or self.k_ring.dtype != torch.bfloat16 or \
                self.v_ring.dtype != torch.bfloat16 or h != self.kv_heads:
            raise ConfigError("KIVI rings must be bf16 [B, Hkv, W, D] (keys) and [B, Hkv, D, W] (values)")
        for t in (self.blocks, self.k_ring, self.v_ring):
            if not t.is_contiguous():
                raise ConfigError("KIVI cache tensors must be contiguous")
        for name in ("keys_quantized", "values_quantized"):
            counts = getattr(self, name)
            if counts.dtype != torch.int32 or counts.shape != (b,):
                raise ConfigError(f"KIVI {name} must be int32 [{b}]")

    def check_flags(self) -> None:
        """The reference's pass-boundary check (techniques/kv_quant/packed.py:175-188): raises ConfigError when a
        quantization since the last check produced a scale or zero point beyond fp16, which the packed pages cannot
        hold, and clears the flag. It reads the device flag, so it waits for the quantizations before it."""
        if int(self.overflow.item()):
            self.overflow.zero_()
            raise ConfigError(
                "a KIVI scale or zero point exceeds the fp16 range of the packed storage; use storage='simulated'")


def _table(block_table: torch.Tensor, batch: int) -> None:
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != batch or \
            block_table.stride(1) != 1:
        raise ConfigError("block_table must be int32 [B, pages] with contiguous rows")


def kivi_append(cache: PagedKIVICache, key: torch.Tensor, value: torch.Tensor, rows: torch.Tensor,
                positions: torch.Tensor) -> None:
    """Writes ``key`` / ``value`` ``[T, Hkv, D]`` (bf16, fp16 or fp32; contiguous channels) into the rings: token ``i``
    is position ``positions[i]`` of row ``rows[i]`` (int32 ``[T]``; negative positions are skipped)."""
    cache.check()
    device = _lib.require_gpu(key, value, rows, positions, cache.k_ring)
    if key.dim() != 3 or key.shape != value.shape or key.shape[1:] != (cache.kv_heads, cache.head_dim):
        raise ConfigError(f"KIVI append takes [T, {cache.kv_heads}, {cache.head_dim}] K/V, got {tuple(key.shape)}")
    if key.stride(-1) != 1 or value.stride(-1) != 1 or key.dtype != value.dtype:
        raise ConfigError("KIVI append takes K/V of one dtype with a contiguous channel axis")
    for t in (rows, positions):
        if t.dtype != torch.int32 or t.shape != (key.shape[0],):
            raise ConfigError("rows and positions must be int32 [T]")
    _lib.call("eco_kivi_ring_write", key.data_ptr(), value.data_ptr(), _lib.fmt(key.dtype), key.stride(0),
              key.stride(1), value.stride(0), value.stride(1), rows.data_ptr(), positions.data_ptr(), key.shape[0],
              cache.k_ring.data_ptr(), cache.v_ring.data_ptr(), cache.batch, cache.kv_heads, cache.head_dim,
              cache.ring, _lib.stream_of(device))


def kivi_quantize(cache: PagedKIVICache, block_table: torch.Tensor, source: torch.Tensor, kind: str,
                  start: torch.Tensor, stop: torch.Tensor, max_tokens: int, source_start: int = 0) -> None:
    """Quantizes tokens ``[start[b], stop[b])`` of every row (int32 ``[B]`` on the device) from ``source``
    ``[B, Hkv, S, D]`` (token ``t`` at index ``t - source_start``) into the pages; ``kind`` is ``"k"`` (ranges of
    whole 32-token groups) or ``"v"``. ``max_tokens`` bounds ``stop - start``."""
    cache.check()
    _table(block_table, cache.batch)
    device = _lib.require_gpu(source, block_table, start, stop, cache.blocks)
    if source.dim() != 4 or source.shape[:2] != (cache.batch, cache.kv_heads) or source.shape[3] != cache.head_dim:
        raise ConfigError(f"KIVI source must be [B, Hkv, S, D], got {tuple(source.shape)}")
    if kind not in ("k", "v"):
        raise ConfigError(f"kind must be 'k' or 'v', not {kind!r}")
    _quantize(cache, block_table, source.data_ptr(), _lib.fmt(source.dtype), source.stride(0), source.stride(1),
              source.stride(2), source.stride(3), source_start, 0, kind, start, stop, max_tokens, device)


def _quantize(cache, block_table, src, fmt, sb, sh, st, sd, src_start, src_ring, kind, start, stop, max_tokens,
              device) -> None:
    _lib.call("eco_kivi_quantize", 0 if kind == "k" else 1, src, fmt, sb, sh, st, sd, src_start, src_ring,
              start.data_ptr(), stop.data_ptr(), cache.blocks.data_ptr(), cache.num_pages, block_table.data_ptr(),
              block_table.stride(0), block_table.shape[1], cache.batch, cache.kv_heads, cache.head_dim, cache.bits,
              cache.group, int(max_tokens), cache.overflow.data_ptr(), _lib.stream_of(device))


def kivi_commit(cache: PagedKIVICache, block_table: torch.Tensor, committed: torch.Tensor,
                max_new: int) -> torch.Tensor:
    """The reference's pass boundary (techniques/kv_quant/kivi.py:191-243): with ``committed`` (int32 ``[B]``)
    tokens per row, quantizes from the rings the keys up to ``(c // R) * R`` and the values up to ``c - R`` that are
    not yet quantized, and advances the counts. ``max_new`` bounds the tokens a row commits since the last call (it
    sizes the launches; the rings must still hold them). Returns the int32 ``[4, B]`` ranges quantized."""
    cache.check()
    headroom = cache.ring - cache.residual
    if int(max_new) > headroom:  # the reference's ring check (techniques/kv_quant/packed.py:180-183)
        raise ConfigError(
            f"a pass of {int(max_new)} tokens is more than the KIVI ring holds beyond the residual ({cache.ring} slots "
            f"= residual_length + headroom {headroom}) and would overwrite entries not quantized yet: increase headroom "
            "or use storage='simulated'")
    _table(block_table, cache.batch)
    device = _lib.require_gpu(committed, block_table, cache.blocks)
    if committed.dtype != torch.int32 or committed.shape != (cache.batch,):
        raise ConfigError(f"committed must be int32 [{cache.batch}]")
    ranges = torch.empty(4, cache.batch, dtype=torch.int32, device=device)
    stream = _lib.stream_of(device)
    _lib.call("eco_kivi_schedule", committed.data_ptr(), cache.residual, cache.group,
              cache.keys_quantized.data_ptr(), cache.values_quantized.data_ptr(), ranges.data_ptr(), cache.batch,
              stream)
    d = cache.head_dim
    keys_new = int(max_new) + cache.residual  # a key block of R tokens completes at once
    _quantize(cache, block_table, cache.k_ring.data_ptr(), _lib.fmt(torch.bfloat16), cache.k_ring.stride(0),
              cache.k_ring.stride(1), d, 1, 0, cache.ring, "k", ranges[0], ranges[1], keys_new, device)
    _quantize(cache, block_table, cache.v_ring.data_ptr(), _lib.fmt(torch.bfloat16), cache.v_ring.stride(0),
              cache.v_ring.stride(1), 1, cache.ring, 0, cache.ring, "v", ranges[2], ranges[3], int(max_new), device)
    return ranges


def kivi_decode_attention(query: torch.Tensor, cache: PagedKIVICache, block_table: torch.Tensor,
                          seq_lens: torch.Tensor, max_seq_len: int, scale: float | None = None,
                          softcap: float | None = None, sinks: torch.Tensor | None = None,
                          out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                          mask: torch.Tensor | None = None) -> torch.Tensor:
    """Attention of ``query`` ``[B, Q, Hq, D]`` (bf16, contiguous channels) over the KIVI cache, ``[B, Q, Hq, D]``
    bf16 out: row ``b`` holds ``seq_lens[b]`` tokens (int32 ``[B]``), its ``Q`` queries the last of them (causal).
    Keys below ``keys_quantized[b]`` and values below ``values_quantized[b]`` are codes, the rest come from the
    rings. ``scale`` defaults to ``1 / sqrt(D)``. ``mask`` (boolean ``[B or 1, Hq or 1, Q or 1, S]``, key ``t`` =
    token ``t``) hides keys on top of the causal limit."""
    cache.check()
    _table(block_table, cache.batch)
    device = _lib.require_gpu(query, cache.blocks, block_table, seq_lens)
    if query.dim() != 4 or query.dtype != torch.bfloat16 or query.stride(-1) != 1:
        raise ConfigError("KIVI decode takes a bf16 query [B, Q, Hq, D] with a contiguous channel axis")
    batch, queries, q_heads, head_dim = query.shape
    if batch != cache.batch or head_dim != cache.head_dim:
        raise ConfigError(f"query {tuple(query.shape)} does not match the cache")
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (batch,):
        raise ConfigError("seq_lens must be int32 [B]")
    if max_seq_len <= 0 or max_seq_len > block_table.shape[1] * KIVI_PAGE:
        raise ConfigError(f"max_seq_len {max_seq_len} must be positive and within the block table")
    if sinks is not None:
        if sinks.numel() != q_heads:
            raise ConfigError(f"{sinks.numel()} sink logits for {q_heads} query heads")
        sinks = sinks.reshape(-1).float().contiguous()
    if out is None:
        out = torch.empty(batch, queries, q_heads, head_dim, dtype=torch.bfloat16, device=device)
    elif out.shape != query.shape or out.dtype != torch.bfloat16 or out.stride(-1) != 1:
        raise ConfigError("out must be bf16 like the query, with a contiguous channel axis")
    need = int(_lib.lib().eco_kivi_decode_workspace_size(batch, queries, q_heads, cache.kv_heads, head_dim,
                                                         int(max_seq_len), cache.bits))
    if workspace is None:
        workspace = cached_workspace(need, counter_bytes(batch, cache.kv_heads), device)
    scale = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)
    bits, mk, words = packed_mask(mask, batch, q_heads, queries)
    _lib.call(
        "eco_kivi_decode", query.data_ptr(), query.stride(0), query.stride(1), query.stride(2),
        cache.blocks.data_ptr(), cache.num_pages, cache.k_ring.data_ptr(), cache.v_ring.data_ptr(), cache.ring,
        cache.keys_quantized.data_ptr(), cache.values_quantized.data_ptr(), block_table.data_ptr(),
        block_table.stride(0), block_table.shape[1], seq_lens.data_ptr(), _lib.ptr(sinks), out.data_ptr(),
        out.stride(0), out.stride(1), out.stride(2), batch, queries, q_heads, cache.kv_heads, head_dim, cache.bits,
        cache.group, int(max_seq_len), scale, float(softcap or 0.0), _lib.ptr(bits), *mk, words,
        workspace.data_ptr(), workspace.numel(),
        _lib.stream_of(device),
    )
    return out


def kivi_gather(cache: PagedKIVICache, block_table: torch.Tensor, keys: int, dtype: torch.dtype = torch.bfloat16
                ) -> tuple[torch.Tensor, torch.Tensor]:
    """The dense view ``[B, Hkv, keys, D]`` of the first ``keys`` tokens of every row: codes dequantized as the
    reference's ``dequantize`` (bf16 of ``code * scale + zero``), the rest from the rings (``KIVIPacked``'s
    materialize, attention/packed.py:66-78). The rings hold the last ``ring`` tokens of a row only."""
    cache.check()
    _table(block_table, cache.batch)
    device = _lib.require_gpu(block_table, cache.blocks)
    shape = (cache.batch, cache.kv_heads, int(keys), cache.head_dim)
    k = torch.empty(shape, dtype=dtype, device=device)
    v = torch.empty(shape, dtype=dtype, device=device)
    if keys > 0:
        _lib.call("eco_kivi_gather", cache.blocks.data_ptr(), cache.num_pages, cache.k_ring.data_ptr(),
                  cache.v_ring.data_ptr(), cache.ring, cache.keys_quantized.data_ptr(),
                  cache.values_quantized.data_ptr(), block_table.data_ptr(), block_table.stride(0),
                  block_table.shape[1], k.data_ptr(), v.data_ptr(), _lib.fmt(dtype), *k.stride()[:3],
                  *v.stride()[:3], cache.batch, cache.kv_heads, int(keys), cache.head_dim, cache.bits, cache.group,
                  _lib.stream_of(device))
    return k, v


def value_group(dim: int, group: int) -> int:
    """Channels per value group: ``group``, or the whole head when ``group`` does not divide it (kivi.py:143-154)."""
    return group if dim % group == 0 else dim


def kivi_fake_quantize(buffer: torch.Tensor, start: int, stop: int, bits: int, group: int, kind: str) -> None:
    """KIVI's simulated storage: slots ``start:stop`` of a dense K or V buffer ``[B, H, S, D]`` (bf16, fp16 or
    fp32, contiguous channels) quantized in place (``kind`` ``"k"``: per channel over groups of ``group`` tokens;
    ``"v"``: per token over groups of :func:`value_group` channels), every element replaced by ``code * scale + low``
    rounded to the buffer's dtype (``KIVICache._quantize``, techniques/kv_quant/kivi.py:257-275)."""
    device = _lib.require_gpu(buffer)
    if buffer.dim() != 4 or buffer.stride(3) != 1:
        raise ConfigError("kivi_fake_quantize takes a [B, H, S, D] buffer with contiguous channels")
    if kind not in ("k", "v"):
        raise ConfigError(f"kind must be 'k' or 'v', not {kind!r}")
    batch, heads, slots, dim = buffer.shape
    g = group if kind == "k" else value_group(dim, group)
    _lib.call("eco_kivi_fake_quantize", buffer.data_ptr(), _lib.fmt(buffer.dtype), buffer.stride(0),
              buffer.stride(1), buffer.stride(2), batch, heads, slots, dim, int(start), int(stop), int(bits), g,
              1 if kind == "k" else 0, _lib.stream_of(device))
