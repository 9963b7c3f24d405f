"""Quest page selection on the GPU (Quest, Tang et al., ICML 2024), over a dense cache and over the paged one.

Mirrors the reference's attention/quest.py and the bound maintenance of techniques/quest/technique.py:

* :func:`page_bounds` is ``page_bounds`` (attention/quest.py:54-65) over a dense key buffer ``[B, H, S, D]`` of any
  dtype, and :func:`bounds_dtype` its result dtype (bf16 for fp8 keys, else the keys' own); :func:`paged_page_bounds`
  computes the same bounds over the paged fp8 / bf16 cache through its block table.
* :func:`select_pages` is ``select_pages`` (attention/quest.py:73-108): the top ``min(pages, max_done)`` committed
  pages of every row and KV head by ``sum_d qsum_d (lo + hi) / 2 + qabs_d (hi - lo) / 2``, in increasing order, then
  ``-1``; ties go to the lower page (torch's order at ties is unspecified). Queries and bounds may be bf16, fp16 or
  fp32.
* :class:`QuestPages` is the packed attachment of format ``"quest"`` (attention/quest.py:112-204): ``select``,
  ``keep`` and ``restrict_mask`` (what an attention function without the kernel hides), ``attend`` over dense K/V
  and ``attend_paged`` over the paged cache.
* :func:`quest_decode_attention` is ``quest_decode_attention`` (attention/quest.py:239-344) over dense K/V: the dense
  decode kernel over the virtual key axis of the selected pages and the dense tail (``eco_quest_decode``);
  :func:`paged_quest_decode_attention` is the same over the paged cache (the paged decode kernel's page list).
* :class:`QuestState` keeps a paged layer's bounds up to date as pages are committed with every count on the device
  (``eco_quest_refresh_bounds``, or folded into the append by ``eco_paged_append_quest``), so that a decode step of
  fixed shapes can be captured in a graph, which the reference's host ``done`` list rules out
  (techniques/quest/technique.py:165-172, 229-259, 311).

Every function runs on the HIP kernels of ``libeconomize_amd.so``; there is no CPU path.
"""

from __future__ import annotations

import math
from collections.abc import Callable
from dataclasses import dataclass

import torch

from . import _lib
from .errors import ConfigError
from .paged import PAGE, PagedKVCache, paged_decode_attention

__all__ = ["QuestPages", "QuestState", "bounds_dtype", "page_bounds", "paged_page_bounds",
           "paged_quest_decode_attention", "quest_decode_attention", "select_pages"]

_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)
_DOT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def bounds_dtype(key_dtype: torch.dtype) -> torch.dtype:
    """The dtype of the page bounds of keys of ``key_dtype``: bf16 for fp8 keys (it holds every fp8 value exactly),
    else the keys' own dtype (attention/quest.py:68-70)."""
    return torch.bfloat16 if key_dtype in _FP8 else key_dtype


def _check_page(page: int, least: int = 16) -> None:
    if page < least or page & (page - 1):
        raise ConfigError(f"quest pages must hold a power of two of at least {least} slots, got {page}")


def page_bounds(keys: torch.Tensor, first: int, last: int, page: int,
                out: tuple[torch.Tensor, torch.Tensor] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Channel-wise smallest and largest key of pages ``first .. last - 1`` of ``keys`` ``[B, H, S, D]``.

    Args:
        keys: Dense keys (bf16, fp16, fp32 or fp8; any strides with a contiguous channel axis).
        first, last: Pages to compute (every row); ``last * page <= S``.
        page: Slots per page (a power of two, at least 16).
        out: ``(kmin, kmax)`` ``[B, H, P >= last, D]`` of :func:`bounds_dtype` to write pages ``first .. last - 1``
            into (the others are left as they are, the incremental bounds of techniques/quest/technique.py:229-259).

    Returns:
        ``(kmin, kmax)``: without ``out``, new ``[B, H, last - first, D]`` tensors of :func:`bounds_dtype` (fp8 keys
        in bf16, which holds them exactly, fp32 keys in fp32 and 16-bit keys in their own dtype).
    """
    _check_page(page)
    device = _lib.require_gpu(keys)
    if keys.dim() != 4 or keys.stride(3) != 1:
        raise ConfigError("page_bounds takes keys [B, H, S, D] with a contiguous channel axis")
    batch, heads, slots, dim = keys.shape
    if not 0 <= first <= last or last * page > slots:
        raise ConfigError(f"quest bounds of pages {first} .. {last} do not fit {slots} slots of {page}")
    dtype = bounds_dtype(keys.dtype)
    if out is None:
        shape = (batch, heads, last - first, dim)
        kmin = torch.empty(shape, dtype=dtype, device=device)
        kmax = torch.empty(shape, dtype=dtype, device=device)
        base = first
    else:
        kmin, kmax = out
        base = 0
        if kmin.shape != kmax.shape or tuple(kmin.shape[:2]) != (batch, heads) or kmin.shape[2] < last or \
                kmin.shape[3] != dim:
            raise ConfigError(f"quest bounds of shape {tuple(kmin.shape)} do not hold {last} pages")
    for t in (kmin, kmax):
        if t.dtype != dtype or t.stride(3) != 1 or t.device != device:
            raise ConfigError(f"quest bounds of {keys.dtype} keys must be {dtype} with a contiguous channel axis")
    if last == first:
        return kmin, kmax
    es = kmin.element_size()
    _lib.call(
        "eco_quest_dense_bounds", keys.data_ptr(), _lib.fmt(keys.dtype), keys.stride(0), keys.stride(1),
        keys.stride(2), slots, first, last, page, kmin.data_ptr() - base * kmin.stride(2) * es,
        kmax.data_ptr() - base * kmax.stride(2) * es, _lib.fmt(dtype), kmin.stride(0), kmin.stride(1), kmin.stride(2),
        batch, heads, dim, _lib.stream_of(device),
    )
    return kmin, kmax


def paged_page_bounds(cache: PagedKVCache, block_table: torch.Tensor, first: int, last: int, page: int = PAGE,
                      out: tuple[torch.Tensor, torch.Tensor] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """:func:`page_bounds` over the paged key cache: Quest pages ``first .. last - 1`` of every row of
    ``block_table`` (int32 ``[B, cache pages per row]``), in bf16 (fp8 keys are decoded exactly).

    Returns:
        ``(kmin, kmax)``; without ``out``, new ``[B, Hkv, last - first, D]`` tensors indexed from ``first``; with it,
        pages ``first .. last - 1`` written into ``out`` (the others left as they are).
    """
    cache.check()
    _check_page(page, PAGE)
    device = _lib.require_gpu(cache.keys, block_table)
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ConfigError("block_table must be int32 [B, pages] with contiguous rows")
    batch = block_table.shape[0]
    if not 0 <= first <= last:
        raise ConfigError(f"quest bounds need 0 <= first <= last, got {first}, {last}")
    if out is None:
        shape = (batch, cache.kv_heads, last - first, cache.head_dim)
        kmin = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        kmax = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        base = first
    else:
        kmin, kmax = out
        base = 0
        if kmin.shape != kmax.shape or kmin.shape[:2] != (batch, cache.kv_heads) or kmin.shape[2] < last:
            raise ConfigError(f"quest bounds of shape {tuple(kmin.shape)} do not hold {last} pages")
    for t in (kmin, kmax):
        if t.dtype != torch.bfloat16 or t.stride(3) != 1 or t.shape[3] != cache.head_dim:
            raise ConfigError("quest bounds must be bf16 [B, Hkv, P, D] with a contiguous channel axis")
    if last == first:
        return kmin, kmax
    # the kernel addresses page p of the output at p * stride: shift the base so that page `first` lands at 0
    kmin_at = kmin.data_ptr() - base * kmin.stride(2) * 2
    kmax_at = kmax.data_ptr() - base * kmax.stride(2) * 2
    _lib.call(
        "eco_quest_page_bounds", cache.keys.data_ptr(), _lib.fmt(cache.dtype), cache.num_pages,
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], first, last, page, kmin_at, kmax_at,
        kmin.stride(0), kmin.stride(1), kmin.stride(2), batch, cache.kv_heads, cache.head_dim, PAGE,
        _lib.stream_of(device),
    )
    return kmin, kmax


def select_pages(query: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, done: torch.Tensor, max_done: int,
                 pages: int, first_page: bool = False) -> torch.Tensor:
    """The committed pages every row and KV head reads.

    Args:
        query: ``[B, Hq, Q, D]`` bf16, fp16 or fp32 (any strides with a contiguous channel axis).
        kmin: ``[B, Hkv, P, D]`` per-page smallest keys (``P >= max_done``; bf16, fp16 or fp32).
        kmax: ``[B, Hkv, P, D]`` the largest keys, like ``kmin``.
        done: int32 ``[B]`` committed pages of every row.
        max_done: ``max(done)``, on the host.
        pages: Pages to select per row and KV head.
        first_page: Always select a row's page 0 (the "first and last pages" variant; the reference's selection,
            the default, has no such rule).

    Returns:
        int32 ``[B, Hkv, pages]``: the selected pages in increasing order, then ``-1``. A row with at most ``pages``
        committed pages selects all of them.
    """
    device = _lib.require_gpu(query, kmin, kmax, done)
    if query.dim() != 4 or query.dtype not in _DOT_DTYPES or query.stride(3) != 1:
        raise ConfigError("quest selection takes a bf16, fp16 or fp32 query [B, Hq, Q, D] with a contiguous channel "
                          "axis")
    batch, q_heads, queries, head_dim = query.shape
    if kmin.dim() != 4 or kmin.shape != kmax.shape or kmin.shape[0] != batch or kmin.shape[3] != head_dim:
        raise ConfigError(f"quest bounds {tuple(kmin.shape)} / {tuple(kmax.shape)} do not match the query")
    kv_heads = kmin.shape[1]
    if q_heads % kv_heads:
        raise ConfigError(f"{q_heads} query heads are not a multiple of {kv_heads} KV heads")
    if kmin.dtype not in _DOT_DTYPES or kmax.dtype != kmin.dtype or kmin.stride() != kmax.stride() or \
            kmin.stride(3) != 1:
        raise ConfigError("quest bounds must be bf16, fp16 or fp32 tensors of one dtype and equal strides")
    if kmin.shape[2] < max_done:
        raise ConfigError(f"quest bounds of {kmin.shape[2]} pages do not cover {max_done} committed ones")
    if done.dtype != torch.int32 or done.shape != (batch,):
        raise ConfigError("done must be int32 [B]")
    out = torch.empty(batch, kv_heads, max(pages, 0), dtype=torch.int32, device=device)
    if pages <= 0:
        return out
    max_done = max(int(max_done), 0)
    need = int(_lib.lib().eco_quest_select_workspace_size(batch, kv_heads, max_done))
    scores = torch.empty(max(need, 4) // 4, dtype=torch.float32, device=device)
    _lib.call(
        "eco_quest_select", query.data_ptr(), _lib.fmt(query.dtype), query.stride(0), query.stride(2),
        query.stride(1), kmin.data_ptr(), kmax.data_ptr(), _lib.fmt(kmin.dtype), kmin.stride(0), kmin.stride(1),
        kmin.stride(2), done.data_ptr(), max_done, pages, int(bool(first_page)), out.data_ptr(), batch, queries,
        q_heads, kv_heads, head_dim, scores.data_ptr(), scores.numel() * 4, _lib.stream_of(device),
    )
    return out


@dataclass
class QuestPages:
    """Page bounds of one layer's committed cache, the packed attachment of format ``"quest"`` (the reference's
    ``QuestPages``, attention/quest.py:112-204).

    Attributes:
        kmin: ``[B, Hkv, P, D]`` channel-wise smallest key of every committed page (rows below ``done[b]`` valid).
        kmax: ``[B, Hkv, P, D]`` the largest keys.
        done: int32 ``[B]`` committed pages of every row; slots from ``done[b] * page`` on are read densely.
        min_done: ``min(done)``, on the host.
        max_done: ``max(done)``, on the host.
        page: Slots per page (a power of two, at least 16).
        pages: Committed pages every row and KV head reads.
        max_queries: Longest query (tokens per row) restricted to the pages; longer ones see every key.
        on_use: Called with ``layer`` whenever an attention function reads the pages (the cache checks that every
            attached layer was read).
        layer: The cache layer.
        first_page: Always select a row's page 0 (off in the reference).
    """

    kmin: torch.Tensor
    kmax: torch.Tensor
    done: torch.Tensor
    min_done: int
    max_done: int
    page: int
    pages: int
    max_queries: int = 1
    on_use: Callable[[int], None] | None = None
    layer: int = 0
    first_page: bool = False
    format: str = "quest"

    def select(self, query: torch.Tensor) -> torch.Tensor:
        """int32 ``[B, Hkv, pages]`` selected pages for ``query`` ``[B, Hq, Q, D]`` (see :func:`select_pages`)."""
        return select_pages(query, self.kmin, self.kmax, self.done, self.max_done, self.pages, self.first_page)

    def keep(self, query: torch.Tensor, slots: int) -> torch.Tensor:
        """Boolean ``[B, Hkv, slots]``: the slots ``query`` reads, its selected pages and every slot from
        ``done[b] * page`` on (attention/quest.py:145-154)."""
        index = self.select(query).long()
        batch, kv_heads, _ = index.shape
        total = -(-slots // self.page)
        # one flag per page, plus a sink column that absorbs the -1 entries
        chosen = torch.zeros(batch, kv_heads, total + 1, dtype=torch.bool, device=index.device)
        chosen.scatter_(-1, torch.where(index < 0, total, index.clamp(max=total)), True)
        keep = chosen[..., :total].repeat_interleave(self.page, dim=-1)[..., :slots]
        tail = (self.done.to(device=index.device, dtype=torch.long) * self.page).view(batch, 1, 1)
        return keep | (torch.arange(slots, device=index.device).view(1, 1, -1) >= tail)

    def _used(self) -> None:
        if self.on_use is not None:
            self.on_use(self.layer)

    def restrict_mask(self, query: torch.Tensor, key: torch.Tensor, mask: torch.Tensor | None,
                      is_causal: bool = False) -> torch.Tensor | None:
        """``mask`` with the unselected pages hidden, for attention functions that read dense K/V
        (attention/quest.py:160-189).

        Args:
            query: ``[B, Hq, Q, D]``.
            key: The dense keys ``[B, Hkv, S, D]``.
            mask: Boolean (``True`` = visible) or additive float mask broadcastable to ``[B, Hq, Q, S]``, or ``None``.
            is_causal: Whether a ``None`` mask stands for a causal one (aligned top-left, as ``sdpa`` reads it).

        Returns:
            A ``[B, Hq, Q, S]`` mask of ``mask``'s kind (boolean for ``None``), or ``mask`` itself for a query longer
            than :attr:`max_queries`.
        """
        batch, q_heads, queries, _ = query.shape
        slots = key.shape[2]
        if queries > self.max_queries:
            return mask
        self._used()
        keep = self.keep(query, slots).repeat_interleave(q_heads // key.shape[1], dim=1)[:, :, None, :]
        if mask is None:
            full = torch.ones(queries, slots, dtype=torch.bool, device=query.device)
            if is_causal:
                full = full.tril()
            return full.expand(batch, q_heads, queries, slots) & keep
        mask = mask[..., :slots].expand(batch, q_heads, queries, slots)
        if mask.dtype == torch.bool:
            return mask & keep
        return mask.masked_fill(~keep, torch.finfo(mask.dtype).min)

    def attend(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
               scale: float, softcap: float | None = None, sinks: torch.Tensor | None = None) -> torch.Tensor:
        """``[B, Q, Hq, Dv]`` attention of ``query`` over dense K/V ``[B, Hkv, S, D]``: the selected pages and the
        tail, or every key for a query longer than :attr:`max_queries` (attention/quest.py:191-204)."""
        from .decode import decode_attention

        if query.shape[2] > self.max_queries:
            return decode_attention(query, key, value, mask, scale, softcap=softcap, sinks=sinks)
        self._used()
        return quest_decode_attention(query, key, value, mask, scale, self, softcap=softcap, sinks=sinks)

    def attend_paged(self, query: torch.Tensor, cache: PagedKVCache, block_table: torch.Tensor,
                     seq_lens: torch.Tensor, max_seq_len: int, scale: float | None = None,
                     softcap: float | None = None, sinks: torch.Tensor | None = None,
                     mask: torch.Tensor | None = None) -> torch.Tensor:
        """:meth:`attend` over the paged cache: ``query`` ``[B, Hq, Q, D]`` (bf16) over the selected pages and the
        tail of every row's ``seq_lens[b]`` tokens, ``[B, Q, Hq, D]`` out."""
        if query.shape[2] > self.max_queries:
            return paged_decode_attention(query.transpose(1, 2), cache, block_table, seq_lens, max_seq_len, scale,
                                          softcap, sinks, mask=mask)
        self._used()
        return paged_quest_decode_attention(query, cache, block_table, seq_lens, max_seq_len, self, scale, softcap,
                                            sinks, mask=mask)


def _check_pages(pages: QuestPages, batch: int, kv_heads: int, head_dim: int, device: torch.device) -> None:
    """The bounds, ``done`` and the host range agree with the query (attention/quest.py:222-236)."""
    _check_page(pages.page)
    shape = (batch, kv_heads, pages.kmin.shape[2], head_dim)
    for name in ("kmin", "kmax"):
        t = getattr(pages, name)
        if tuple(t.shape) != shape or t.device != device:
            raise ConfigError(f"quest {name} is {tuple(t.shape)} on {t.device}, expected {shape} on {device}")
    if pages.kmin.shape[2] < pages.max_done:
        raise ConfigError(f"quest bounds of {pages.kmin.shape[2]} pages do not cover {pages.max_done} committed ones")
    if tuple(pages.done.shape) != (batch,) or pages.done.dtype != torch.int32 or pages.done.device != device:
        raise ConfigError(f"quest done is {tuple(pages.done.shape)} {pages.done.dtype}, expected ({batch},) int32")
    if not 0 <= pages.min_done <= pages.max_done:
        raise ConfigError(f"quest done range {pages.min_done}..{pages.max_done} is empty")


def quest_decode_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
                           scale: float, pages: QuestPages, softcap: float | None = None,
                           sinks: torch.Tensor | None = None, out: torch.Tensor | None = None, launch: object = None,
                           index: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention over the selected pages and the dense tail of dense K/V (attention/quest.py:239-344).

    Args:
        query: ``[B, Hq, Q, D]``, bf16, fp16 or fp32.
        key: Dense ``[B, Hkv, S, D]`` in the query's dtype or an fp8 dtype.
        value: Dense ``[B, Hkv, S, Dv]``, like ``key``.
        mask: Boolean ``[B, 1 or Hq, Q, S]`` over the slots, or ``None``.
        scale: Multiplier of the scores.
        pages: The page bounds (see :class:`QuestPages`).
        softcap: Optional tanh soft cap of the scaled scores.
        sinks: Optional ``[Hq]`` attention-sink logits.
        out: Optional ``[B, Q, Hq, Dv]`` output buffer.
        launch: The reference's launch override; the plan here is a function of the shapes, so it is ignored.
        index: Selected pages (int32 ``[B, Hkv, pages]``) to use instead of :meth:`QuestPages.select`'s.

    Returns:
        ``[B, Q, Hq, Dv]`` in the query's dtype.
    """
    from .decode import FP8_DTYPES, _channel_contiguous, _workspace, mask_operand, sinks_operand

    del launch
    device = _lib.require_gpu(query, key, value)
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ConfigError("quest_decode_attention takes [B, Hq, Q, D] queries and [B, Hkv, S, D] keys and values")
    batch, q_heads, queries, head_dim = query.shape
    _, kv_heads, keys, _ = key.shape
    head_dv = value.shape[-1]
    if key.shape[:3] != value.shape[:3] or key.shape[0] != batch or key.shape[3] != head_dim:
        raise ConfigError(f"K {tuple(key.shape)} / V {tuple(value.shape)} do not match the query {tuple(query.shape)}")
    if q_heads % kv_heads:
        raise ConfigError(f"{q_heads} query heads are not a multiple of {kv_heads} KV heads")
    if query.dtype not in _DOT_DTYPES:
        raise ConfigError(f"quest_decode_attention does not support {query.dtype} queries")
    if key.dtype in FP8_DTYPES:
        if value.dtype != key.dtype:
            raise ConfigError(f"K/V dtypes {key.dtype} / {value.dtype} differ")
    elif key.dtype != query.dtype or value.dtype != key.dtype:
        raise ConfigError(f"K/V dtype {key.dtype} / {value.dtype} does not match the query's {query.dtype}")
    _check_pages(pages, batch, kv_heads, head_dim, device)
    if pages.max_done * pages.page > keys:
        raise ConfigError(f"quest bounds of {pages.max_done} pages do not fit {keys} slots")
    if index is None:
        index = pages.select(query)
    if tuple(index.shape) != (batch, kv_heads, pages.pages) or index.dtype != torch.int32:
        raise ConfigError(f"quest index is {tuple(index.shape)} {index.dtype}, expected int32 {pages.pages} pages")
    index = index if index.stride(2) == 1 else index.contiguous()
    m, mask_strides = mask_operand(mask, keys)
    sinks = sinks_operand(sinks, q_heads)
    if out is not None and (out.shape != (batch, queries, q_heads, head_dv) or out.dtype != query.dtype or
                            out.stride(-1) != 1):
        raise ConfigError("out must be [B, Q, Hq, Dv] in the query's dtype with a contiguous last axis")
    if keys == 0:
        return torch.zeros(batch, queries, q_heads, head_dv, dtype=query.dtype, device=device) if out is None \
            else out.zero_()
    query, key, value = _channel_contiguous(query), _channel_contiguous(key), _channel_contiguous(value)
    if out is None:
        out = torch.empty(batch, queries, q_heads, head_dv, dtype=query.dtype, device=device)
    need = int(_lib.lib().eco_quest_decode_workspace_size(batch, queries, q_heads, kv_heads, keys, pages.pages,
                                                            pages.page, pages.min_done, head_dim, head_dv))
    if need == 0:
        raise ConfigError(f"quest_decode_attention supports head dims up to 512, got {head_dim} / {head_dv}")
    ws = _workspace(need, device, batch, queries, q_heads, kv_heads)
    _lib.call(
        "eco_quest_decode", query.data_ptr(), _lib.fmt(query.dtype), query.stride(0), query.stride(1),
        query.stride(2), key.data_ptr(), value.data_ptr(), _lib.fmt(key.dtype), key.stride(0), key.stride(1),
        key.stride(2), value.stride(0), value.stride(1), value.stride(2), None, None, index.data_ptr(),
        index.stride(0), index.stride(1), pages.pages, pages.done.data_ptr(), pages.page, int(pages.min_done),
        _lib.ptr(m), *mask_strides, _lib.ptr(sinks), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        batch, queries, q_heads, kv_heads, keys, head_dim, head_dv,
        float(scale if scale is not None else 1 / math.sqrt(head_dim)), float(softcap or 0.0), ws.data_ptr(),
        ws.numel(), _lib.stream_of(device),
    )
    return out


def paged_quest_decode_attention(query: torch.Tensor, cache: PagedKVCache, block_table: torch.Tensor,
                                 seq_lens: torch.Tensor, max_seq_len: int, pages: QuestPages,
                                 scale: float | None = None, softcap: float | None = None,
                                 sinks: torch.Tensor | None = None, out: torch.Tensor | None = None,
                                 index: torch.Tensor | None = None, mask: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`quest_decode_attention` over the paged cache (the paged decode kernel with a page list).

    Args:
        query: bf16 ``[B, Hq, Q, D]``.
        cache, block_table, seq_lens, max_seq_len: the paged cache (see
            :func:`~economize_amd.paged.paged_decode_attention`).
        pages: The page bounds.
        scale: Multiplier of the scores (``1 / sqrt(D)`` by default).
        softcap: Optional tanh soft cap.
        sinks: Optional ``[Hq]`` attention-sink logits.
        out: Optional ``[B, Q, Hq, D]`` output buffer.
        index: Selected pages (int32 ``[B, Hkv, pages]``) to use instead of :meth:`QuestPages.select`'s.
        mask: Optional boolean attention mask (see :func:`~economize_amd.paged.paged_decode_attention`).

    Returns:
        bf16 ``[B, Q, Hq, D]``.
    """
    _check_page(pages.page, PAGE)
    batch = query.shape[0]
    if tuple(pages.done.shape) != (batch,) or pages.done.dtype != torch.int32:
        raise ConfigError(f"quest done is {tuple(pages.done.shape)} {pages.done.dtype}, expected ({batch},) int32")
    if not 0 <= pages.min_done <= pages.max_done:
        raise ConfigError(f"quest done range {pages.min_done}..{pages.max_done} is empty")
    if index is None:
        index = pages.select(query)
    if tuple(index.shape) != (batch, cache.kv_heads, pages.pages) or index.dtype != torch.int32:
        raise ConfigError(f"quest index is {tuple(index.shape)} {index.dtype}, expected int32 {pages.pages} pages")
    scale = 1.0 / math.sqrt(query.shape[-1]) if scale is None else scale
    return paged_decode_attention(query.transpose(1, 2), cache, block_table, seq_lens, max_seq_len, scale, softcap,
                                  sinks, out, page_list=index.contiguous(), done=pages.done,
                                  list_page_size=pages.page, mask=mask)


class QuestState:
    """One layer's Quest metadata with every count on the device: bounds ``[B, Hkv, max_pages, D]`` (bf16), the
    pages of every (row, KV head) whose bounds are final, and ``done`` ``[B]`` (committed Quest pages).
    :meth:`refresh` computes the bounds of the pages committed since the last refresh from device committed lengths
    (the reference's ``pass_begin`` + ``_layer_bounds``, techniques/quest/technique.py:165-172, 229-259), and
    :meth:`pages_handle` hands the selection and the attention ``max_done = max_pages``: the calls of a decode step
    then have fixed shapes and no host value that changes from step to step. Pages past a row's ``done`` score
    ``-inf``, so the selection equals the one with the batch's true ``max(done)`` whenever it exceeds ``pages``; a row
    with at most ``pages`` committed pages selects all of them (dense attention, in another key order).
    """

    def __init__(self, batch: int, kv_heads: int, head_dim: int, max_pages: int, page: int, pages: int,
                 device: torch.device | str, max_queries: int = 1, first_page: bool = False) -> None:
        _check_page(page, PAGE)
        if max_pages <= 0 or pages <= 0:
            raise ConfigError(f"quest state needs positive max_pages and pages, got {max_pages}, {pages}")
        shape = (batch, kv_heads, max_pages, head_dim)
        self.kmin = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.kmax = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.valid = torch.zeros(batch * kv_heads, dtype=torch.int32, device=device)
        self.done = torch.zeros(batch, dtype=torch.int32, device=device)
        self.counters = torch.zeros(batch * kv_heads, dtype=torch.int32, device=device)  # zero between calls
        self.page, self.pages, self.max_pages, self.max_queries = page, pages, max_pages, max_queries
        self.first_page = first_page

    def reset(self) -> None:
        """Forget every page (a new generation in the same buffers)."""
        self.valid.zero_()
        self.done.zero_()

    def _check(self, cache: PagedKVCache, block_table: torch.Tensor, committed: torch.Tensor) -> torch.device:
        cache.check()
        device = _lib.require_gpu(cache.keys, block_table, committed)
        batch = self.done.shape[0]
        if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1 or \
                block_table.shape[0] != batch:
            raise ConfigError(f"block_table must be int32 [{batch}, pages] with contiguous rows")
        if committed.dtype != torch.int32 or committed.shape != (batch,) or not committed.is_contiguous():
            raise ConfigError(f"committed must be a contiguous int32 [{batch}]")
        if self.kmin.shape[1] != cache.kv_heads or self.kmin.shape[3] != cache.head_dim:
            raise ConfigError("the quest state was made for another number of KV heads or head dim")
        return device

    def refresh(self, cache: PagedKVCache, block_table: torch.Tensor, committed: torch.Tensor) -> None:
        """Bounds of the pages below ``committed`` (int32 ``[B]`` tokens, on the device) not computed yet; ``done``
        becomes ``committed // page`` (at most ``max_pages``)."""
        device = self._check(cache, block_table, committed)
        batch = self.done.shape[0]
        _lib.call(
            "eco_quest_refresh_bounds", cache.keys.data_ptr(), _lib.fmt(cache.dtype), cache.num_pages,
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1], committed.data_ptr(),
            self.valid.data_ptr(), self.done.data_ptr(), self.page, self.kmin.data_ptr(), self.kmax.data_ptr(),
            self.kmin.stride(0), self.kmin.stride(1), self.kmin.stride(2), self.max_pages, batch, cache.kv_heads,
            cache.head_dim, PAGE, _lib.stream_of(device),
        )

    def append(self, cache: PagedKVCache, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor,
               block_table: torch.Tensor, committed: torch.Tensor) -> None:
        """:func:`~economize_amd.paged.paged_append` of ``key`` / ``value`` ``[T, Hkv, D]`` at ``slot_mapping`` and
        :meth:`refresh` to ``committed`` in one launch (``eco_paged_append_quest``); the new tokens must lie at or
        past the committed ones. ``T`` may be 0."""
        self._check(cache, block_table, committed)
        device = _lib.require_gpu(key, value, slot_mapping, cache.keys)
        if key.dim() != 3 or key.shape != value.shape or key.shape[1:] != (cache.kv_heads, cache.head_dim):
            raise ConfigError(f"append takes [T, {cache.kv_heads}, {cache.head_dim}] K/V, got {tuple(key.shape)}")
        if key.stride(-1) != 1 or value.stride(-1) != 1 or key.dtype != value.dtype:
            raise ConfigError("append takes K/V of one dtype with a contiguous channel axis")
        if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (key.shape[0],):
            raise ConfigError("slot_mapping must be int32 [T]")
        batch = self.done.shape[0]
        _lib.call(
            "eco_paged_append_quest", key.data_ptr(), value.data_ptr(), _lib.fmt(key.dtype), key.stride(0),
            key.stride(1), value.stride(0), value.stride(1), slot_mapping.data_ptr(), key.shape[0],
            cache.keys.data_ptr(), cache.values.data_ptr(), cache.num_pages, cache.kv_heads, cache.head_dim, PAGE,
            _lib.fmt(cache.dtype), _lib.ptr(cache.k_scale), _lib.ptr(cache.v_scale), block_table.data_ptr(),
            block_table.stride(0), block_table.shape[1], committed.data_ptr(), self.valid.data_ptr(),
            self.done.data_ptr(), self.counters.data_ptr(), self.page, self.kmin.data_ptr(), self.kmax.data_ptr(),
            self.kmin.stride(0), self.kmin.stride(1), self.kmin.stride(2), self.max_pages, batch,
            _lib.stream_of(device),
        )

    def pages_handle(self, on_use: Callable[[int], None] | None = None, layer: int = 0) -> QuestPages:
        """The layer's :class:`QuestPages` with the device ``done`` and ``max_done = max_pages``."""
        return QuestPages(self.kmin, self.kmax, self.done, 0, self.max_pages, self.page, self.pages,
                          max_queries=self.max_queries, on_use=on_use, layer=layer, first_page=self.first_page)
