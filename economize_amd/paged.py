"""Paged fp8 / bf16 KV cache: quantize-and-append, per-head scales and split-K decode attention on the GPU.

The reference keeps fp8 entries in a contiguous slot buffer (techniques/kv_quant/fp8.py:143-217, and
kv_fp8_fused/fused.py:52-63 hands them to the kernel); this module holds them in 16-token pages behind a block table
(vLLM's paged-attention layout, see :class:`PagedKVCache`) and runs the same arithmetic:

* :func:`paged_append` is ``fp8_encode`` (fp8.py:81-86) plus the slot write (modules/kv_cache.py:30-41);
* :func:`head_scales` is ``static_scales`` (fp8.py:130-133) over each KV head's absolute maximum;
* :func:`paged_decode_attention` is ``decode_attention`` (attention/decode.py:252-324) over the pages, and with a
  page list ``quest_decode_attention`` (attention/quest.py:239-344).

Every function runs on the HIP kernels of ``libeconomize_amd.so``; there is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .errors import ConfigError

__all__ = [
    "PAGE", "PagedKVCache", "head_scales", "new_workspace", "packed_mask", "paged_append", "paged_decode_attention",
    "paged_gather", "workspace_size",
]

#: Tokens per page.
PAGE = 16

_CACHE_DTYPES = (torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2)


@dataclass
class PagedKVCache:
    """One layer's paged K/V.

    Attributes:
        keys: ``[pages, Hkv, D / X, 16, X]`` (``X = 16 / element bytes``) in bf16 or an fp8 dtype.
        values: ``[pages, Hkv, D, 16]`` in the same dtype.
        k_scale: fp32 ``[Hkv]`` per-head key scales of an fp8 cache (``None``: unscaled).
        v_scale: fp32 ``[Hkv]`` per-head value scales.
    """

    keys: torch.Tensor
    values: torch.Tensor
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None

    @classmethod
    def empty(cls, pages: int, kv_heads: int, head_dim: int, dtype: torch.dtype, device: torch.device | str,
              k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> PagedKVCache:
        if dtype not in _CACHE_DTYPES:
            raise ConfigError(f"paged KV caches hold bf16 or fp8, not {dtype}")
        x = 16 // torch.empty((), dtype=dtype).element_size()
        if head_dim % x:
            raise ConfigError(f"head dim {head_dim} is not a multiple of {x}")
        keys = torch.zeros(pages, kv_heads, head_dim // x, PAGE, x, dtype=dtype, device=device)
        values = torch.zeros(pages, kv_heads, head_dim, PAGE, dtype=dtype, device=device)
        return cls(keys, values, k_scale, v_scale)

    @property
    def dtype(self) -> torch.dtype:
        return self.keys.dtype

    @property
    def num_pages(self) -> int:
        return self.keys.shape[0]

    @property
    def kv_heads(self) -> int:
        return self.keys.shape[1]

    @property
    def head_dim(self) -> int:
        return self.values.shape[2]

    def check(self) -> None:
        if self.keys.dtype not in _CACHE_DTYPES or self.values.dtype != self.keys.dtype:
            raise ConfigError(f"paged K/V dtypes {self.keys.dtype} / {self.values.dtype}")
        pages, heads, runs, page, x = self.keys.shape
        if page != PAGE or x * self.keys.element_size() != 16 or runs * x != self.head_dim:
            raise ConfigError(f"paged keys of shape {tuple(self.keys.shape)} do not match the layout")
        if tuple(self.values.shape) != (pages, heads, self.head_dim, PAGE):
            raise ConfigError(f"paged values of shape {tuple(self.values.shape)} do not match the keys")
        if not (self.keys.is_contiguous() and self.values.is_contiguous()):
            raise ConfigError("paged caches must be contiguous")
        for name in ("k_scale", "v_scale"):
            s = getattr(self, name)
            if s is not None:
                if self.dtype == torch.bfloat16:
                    raise ConfigError("a bf16 cache takes no scales")
                if s.dtype != torch.float32 or s.numel() != heads or not s.is_contiguous():
                    raise ConfigError(f"{name} must be contiguous fp32 [{heads}]")


def paged_append(cache: PagedKVCache, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Quantize ``key``/``value`` ``[T, Hkv, D]`` (bf16, fp16 or fp32) into the cache at ``slot_mapping`` ``[T]``
    (int32, ``page * 16 + position``; negative slots are skipped)."""
    cache.check()
    device = _lib.require_gpu(key, value, slot_mapping, cache.keys)
    if key.dim() != 3 or key.shape != value.shape or key.shape[1:] != (cache.kv_heads, cache.head_dim):
        raise ConfigError(f"append takes [T, {cache.kv_heads}, {cache.head_dim}] K/V, got {tuple(key.shape)}")
    if key.stride(-1) != 1 or value.stride(-1) != 1 or key.dtype != value.dtype:
        raise ConfigError("append takes K/V of one dtype with a contiguous channel axis")
    if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (key.shape[0],):
        raise ConfigError("slot_mapping must be int32 [T]")
    _lib.call(
        "eco_paged_append", key.data_ptr(), value.data_ptr(), _lib.fmt(key.dtype), key.stride(0), key.stride(1),
        value.stride(0), value.stride(1), slot_mapping.data_ptr(), key.shape[0], cache.keys.data_ptr(),
        cache.values.data_ptr(), cache.num_pages, cache.kv_heads, cache.head_dim, PAGE, _lib.fmt(cache.dtype),
        _lib.ptr(cache.k_scale), _lib.ptr(cache.v_scale), _lib.stream_of(device),
    )


def head_scales(x: torch.Tensor, dtype: torch.dtype = torch.float8_e4m3fn) -> torch.Tensor:
    """fp32 ``[H]``: each head's absolute maximum of ``x`` ``[B, H, S, D]`` over the fp8 format's maximum, 1 where
    the head is all zero (the ``static_scales`` rule, fp8.py:130-133)."""
    device = _lib.require_gpu(x)
    if x.dim() != 4:
        raise ConfigError("head_scales takes [B, H, S, D]")
    b, h, s, d = x.shape
    absmax = torch.zeros(h, dtype=torch.int32, device=device)
    scales = torch.empty(h, dtype=torch.float32, device=device)
    stream = _lib.stream_of(device)
    _lib.call("eco_kv_head_absmax", x.data_ptr(), _lib.fmt(x.dtype), b, h, s, d, *x.stride(), absmax.data_ptr(),
              stream)
    _lib.call("eco_fp8_scales_from_absmax", absmax.data_ptr(), h, _lib.fmt(dtype), scales.data_ptr(), stream)
    return scales


def workspace_size(batch: int, queries: int, q_heads: int, kv_heads: int, head_dim: int, max_seq_len: int,
                   n_sel: int = 0, dtype: torch.dtype = torch.float8_e4m3fn, list_page_size: int = PAGE) -> int:
    """Bytes of scratch :func:`paged_decode_attention` needs for this shape and cache dtype (``n_sel`` listed pages
    of ``list_page_size`` tokens)."""
    return int(_lib.lib().eco_paged_decode_workspace_size(batch, queries, q_heads, kv_heads, head_dim, max_seq_len,
                                                          n_sel, list_page_size, _lib.fmt(dtype)))


def new_workspace(nbytes: int, device: torch.device | str) -> torch.Tensor:
    """A workspace for :func:`paged_decode_attention`: zeroed, since the row counters at its start must be zero when a
    call starts. A call leaves its counters zero but may write anything after them: a workspace passed to calls with
    more rows times KV heads than the previous call needs the bytes between cleared first (:class:`CachedWorkspace`
    does this for the workspace used when none is passed). One workspace serves one stream at a time."""
    return torch.zeros(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def counter_bytes(batch: int, kv_heads: int) -> int:
    """Bytes of the row counters at the start of a decode workspace (int32 per row and KV head, 256-byte aligned).
    They must be zero when a call starts; a call leaves them zero and may write anything after them."""
    return (4 * batch * kv_heads + 255) // 256 * 256


class CachedWorkspace:
    """A workspace reused across calls of any shape on one stream, grown on demand. It tracks the prefix known to be
    zero: a call leaves its counters zero and may dirty everything after them, so a later call with more counters
    first clears the bytes between."""

    def __init__(self) -> None:
        self.buffer: torch.Tensor | None = None
        self.zero_prefix = 0

    def take(self, nbytes: int, counters: int, device: torch.device) -> torch.Tensor:
        if self.buffer is None or self.buffer.numel() < nbytes:
            size = max(nbytes, 2 * (self.buffer.numel() if self.buffer is not None else 0))
            self.buffer = new_workspace(size, device)
            self.zero_prefix = self.buffer.numel()
        if counters > self.zero_prefix:
            self.buffer[self.zero_prefix:counters].zero_()
        self.zero_prefix = counters
        return self.buffer


_workspaces: dict[tuple[torch.device, int], CachedWorkspace] = {}


def packed_mask(mask: torch.Tensor | None, batch: int, q_heads: int, queries: int
                ) -> tuple[torch.Tensor | None, tuple[int, int, int], int]:
    """A boolean attention mask ``[B or 1, Hq or 1, Q or 1, S]`` (``True`` = visible; key ``t`` of the mask is token
    ``t`` of every row) packed for the paged kernels: int32 words ``[B or 1, Hq or 1, Q or 1, ceil(S / 32)]`` (bit
    ``t % 32`` of word ``t / 32``), their ``(batch, head, query)`` word strides (0 on a broadcast axis) and the words
    per row; ``(None, (0, 0, 0), 0)`` without a mask."""
    if mask is None:
        return None, (0, 0, 0), 0
    if mask.dtype != torch.bool or mask.dim() != 4:
        raise ConfigError("the attention mask must be boolean [B or 1, Hq or 1, Q or 1, S]")
    bm, hm, qm, keys = mask.shape
    if bm not in (1, batch) or hm not in (1, q_heads) or qm not in (1, queries) or keys == 0:
        raise ConfigError(f"mask {tuple(mask.shape)} does not broadcast to [{batch}, {q_heads}, {queries}, S]")
    device = _lib.require_gpu(mask)
    words = -(-keys // 32)
    bits = torch.empty(bm, hm, qm, words, dtype=torch.int32, device=device)
    m = mask.view(torch.uint8)
    _lib.call("eco_mask_bits", m.data_ptr(), *m.stride(), bm, hm, qm, keys, bits.data_ptr(), words,
              _lib.stream_of(device))
    strides = (hm * qm * words if bm > 1 else 0, qm * words if hm > 1 else 0, words if qm > 1 else 0)
    return bits, strides, words


def cached_workspace(nbytes: int, counters: int, device: torch.device) -> torch.Tensor:
    """The workspace of ``device``'s current stream used when the caller passes none (see :class:`CachedWorkspace`)."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    return _workspaces.setdefault(key, CachedWorkspace()).take(nbytes, counters, device)


def paged_decode_attention(
    query: torch.Tensor,
    cache: PagedKVCache,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    max_seq_len: int,
    scale: float | None = None,
    softcap: float | None = None,
    sinks: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    page_list: torch.Tensor | None = None,
    done: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    list_page_size: int = PAGE,
    mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """Attention of ``query`` ``[B, Q, Hq, D]`` (bf16, or fp16 over an fp8 cache without a page list; channel-contiguous)
    over the paged cache, ``[B, Q, Hq, D]`` out in the query's dtype.

    Row ``b`` holds ``seq_lens[b]`` tokens (int32 ``[B]`` on the device; ``max_seq_len`` bounds them on the host and
    sizes the launch), its ``Q`` queries the last of them: query ``qi`` sees tokens ``< seq_lens[b] - Q + qi + 1``.
    ``block_table`` is int32 ``[B, pages per row]``. ``scale`` defaults to ``1 / sqrt(D)``.

    With ``page_list`` (int32 ``[B, Hkv, n_sel]``, pages of ``list_page_size`` tokens, ``-1`` = none) and ``done``
    (int32 ``[B]``, in the same pages) the keys read are the listed pages below ``done[b]`` and every token from page
    ``done[b]`` on (Quest's gathered attention).
    ``workspace`` (from :func:`new_workspace`, at least :func:`workspace_size` bytes) defaults to a cached one per
    device and stream. ``mask`` (boolean ``[B or 1, Hq or 1, Q or 1, S]``, key ``t`` = token ``t`` of the row, as the
    reference's decode_attention takes it) hides keys on top of the causal limit.
    """
    cache.check()
    device = _lib.require_gpu(query, cache.keys, block_table, seq_lens)
    if query.dim() != 4 or query.dtype not in (torch.bfloat16, torch.float16) or query.stride(-1) != 1:
        raise ConfigError("paged decode takes a bf16 or fp16 query [B, Q, Hq, D] with a contiguous channel axis")
    if query.dtype == torch.float16 and (cache.dtype == torch.bfloat16 or page_list is not None):
        raise ConfigError("paged decode takes fp16 queries over an fp8 cache without a page list")
    batch, queries, q_heads, head_dim = query.shape
    if head_dim != cache.head_dim:
        raise ConfigError(f"query head dim {head_dim} != cache head dim {cache.head_dim}")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != batch:
        raise ConfigError("block_table must be int32 [B, pages]")
    if block_table.stride(1) != 1:
        raise ConfigError("block_table rows must be contiguous")
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (batch,):
        raise ConfigError("seq_lens must be int32 [B]")
    if max_seq_len > block_table.shape[1] * PAGE:
        raise ConfigError(f"max_seq_len {max_seq_len} exceeds the block table's {block_table.shape[1]} pages")
    n_sel = 0
    if page_list is not None:
        if done is None or page_list.dtype != torch.int32 or page_list.dim() != 3 or page_list.stride(2) != 1:
            raise ConfigError("page_list must be int32 [B, Hkv, n] (contiguous last axis) with done int32 [B]")
        if page_list.shape[:2] != (batch, cache.kv_heads) or done.dtype != torch.int32 or done.shape != (batch,):
            raise ConfigError("page_list / done shapes do not match the batch and KV heads")
        n_sel = page_list.shape[2]
    if sinks is not None:
        if sinks.numel() != q_heads:
            raise ConfigError(f"{sinks.numel()} sink logits for {q_heads} query heads")
        sinks = sinks.reshape(-1).float().contiguous()
    if out is None:
        out = torch.empty(batch, queries, q_heads, head_dim, dtype=query.dtype, device=device)
    elif out.shape != query.shape or out.dtype != query.dtype or out.stride(-1) != 1:
        raise ConfigError("out must be like the query (shape and dtype), with a contiguous channel axis")
    if max_seq_len <= 0:
        raise ConfigError("max_seq_len must be positive")
    if list_page_size < PAGE or list_page_size % PAGE:
        raise ConfigError(f"listed pages must hold a positive multiple of {PAGE} tokens, not {list_page_size}")
    need = workspace_size(batch, queries, q_heads, cache.kv_heads, head_dim, max_seq_len, n_sel, cache.dtype,
                          list_page_size)
    if workspace is None:
        workspace = cached_workspace(need, counter_bytes(batch, cache.kv_heads), device)
    scale = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)
    bits, mk, words = packed_mask(mask, batch, q_heads, queries)
    _lib.call(
        "eco_paged_decode",
        query.data_ptr(), _lib.fmt(query.dtype), query.stride(0), query.stride(1), query.stride(2),
        cache.keys.data_ptr(), cache.values.data_ptr(), _lib.fmt(cache.dtype), cache.num_pages,
        _lib.ptr(cache.k_scale), _lib.ptr(cache.v_scale),
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], seq_lens.data_ptr(),
        _lib.ptr(page_list), page_list.stride(0) if page_list is not None else 0,
        page_list.stride(1) if page_list is not None else 0, n_sel, int(list_page_size), _lib.ptr(done),
        _lib.ptr(sinks),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        batch, queries, q_heads, cache.kv_heads, head_dim, PAGE, int(max_seq_len), scale, float(softcap or 0.0),
        _lib.ptr(bits), *mk, words, workspace.data_ptr(), workspace.numel(), _lib.stream_of(device),
    )
    return out


def paged_gather(cache: PagedKVCache, block_table: torch.Tensor, keys: int, dtype: torch.dtype = torch.bfloat16
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """The dense view ``[B, Hkv, keys, D]`` (``dtype``: bf16, fp16 or fp32) of the first ``keys`` tokens of every
    row: fp8 decoded exactly and times the per-head scales, 0 past a row's table (``materialize()`` of
    attention/packed.py:66-78 for this cache)."""
    cache.check()
    device = _lib.require_gpu(cache.keys, block_table)
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ConfigError("block_table must be int32 [B, pages] with contiguous rows")
    batch = block_table.shape[0]
    shape = (batch, cache.kv_heads, int(keys), cache.head_dim)
    k = torch.empty(shape, dtype=dtype, device=device)
    v = torch.empty(shape, dtype=dtype, device=device)
    if keys > 0:
        _lib.call("eco_paged_gather", cache.keys.data_ptr(), cache.values.data_ptr(), _lib.fmt(cache.dtype),
                  cache.num_pages, _lib.ptr(cache.k_scale), _lib.ptr(cache.v_scale), block_table.data_ptr(),
                  block_table.stride(0), block_table.shape[1], k.data_ptr(), v.data_ptr(), _lib.fmt(dtype),
                  *k.stride()[:3], *v.stride()[:3], batch, cache.kv_heads, int(keys), cache.head_dim, PAGE,
                  _lib.stream_of(device))
    return k, v
