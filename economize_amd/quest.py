"""Quest page selection over the paged KV cache on the GPU (Quest, Tang et al., ICML 2024).

Mirrors the reference's attention/quest.py and the bound maintenance of techniques/quest/technique.py:

* :func:`page_bounds` is ``page_bounds`` (attention/quest.py:54-65) over the paged key cache: the channel-wise
  smallest and largest stored key of every Quest page, in bf16 (fp8 keys are decoded exactly).
* :func:`select_pages` is ``select_pages`` (attention/quest.py:73-108): the top ``min(pages, max_done)`` committed
  pages of every row and KV head by ``sum_d qsum_d (lo + hi) / 2 + qabs_d (hi - lo) / 2``, in increasing order, then
  ``-1``; ties go to the lower page (torch's order at ties is unspecified).
* :class:`QuestPages` carries one layer's bounds like the reference's ``QuestPages`` (attention/quest.py:112-204), and
  :func:`quest_decode_attention` attends over the selected pages and the dense tail from page ``done[b]`` on
  (attention/quest.py:239-344) with the paged decode kernel.
* :class:`QuestState` keeps a layer's bounds up to date as pages are committed with every count on the device
  (``eco_quest_refresh_bounds``), so that a decode step of fixed shapes can be captured in a graph, which the
  reference's host ``done`` list rules out (techniques/quest/technique.py:165-172, 229-259, 311).

Every function runs on the HIP kernels of ``libeconomize_amd.so``; there is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .errors import ConfigError
from .paged import PAGE, PagedKVCache, paged_decode_attention

__all__ = ["QuestPages", "QuestState", "bounds_dtype", "page_bounds", "quest_decode_attention", "select_pages"]


def bounds_dtype(key_dtype: torch.dtype) -> torch.dtype:
    """The dtype of the page bounds of a cache of ``key_dtype``: bf16 (it holds every fp8 value exactly)."""
    return torch.bfloat16


def _check_page(page: int) -> None:
    if page < PAGE or page & (page - 1):
        raise ConfigError(f"quest pages must hold a power of two of at least {PAGE} slots, got {page}")


def page_bounds(cache: PagedKVCache, block_table: torch.Tensor, first: int, last: int, page: int = PAGE,
                out: tuple[torch.Tensor, torch.Tensor] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Channel-wise smallest and largest key of Quest pages ``first .. last - 1`` of every row.

    Args:
        cache: The layer's paged cache.
        block_table: int32 ``[B, cache pages per row]``.
        first, last: Quest pages to compute (every row).
        page: Tokens per Quest page (a power of two, at least 16).
        out: ``(kmin, kmax)`` bf16 ``[B, Hkv, P >= last, D]`` to write into (pages outside ``[first, last)`` are
            left as they are, like the reference's incremental bounds, techniques/quest/technique.py:229-259).

    Returns:
        ``(kmin, kmax)``; without ``out``, new ``[B, Hkv, last - first, D]`` tensors indexed from ``first``.
    """
    cache.check()
    _check_page(page)
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
        query: bf16 ``[B, Hq, Q, D]`` (any strides with a contiguous channel axis).
        kmin: bf16 ``[B, Hkv, P, D]`` per-page smallest keys (``P >= max_done``).
        kmax: bf16 ``[B, Hkv, P, D]`` the largest keys.
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
    if query.dim() != 4 or query.dtype != torch.bfloat16 or query.stride(3) != 1:
        raise ConfigError("quest selection takes a bf16 query [B, Hq, Q, D] with a contiguous channel axis")
    batch, q_heads, queries, head_dim = query.shape
    if kmin.dim() != 4 or kmin.shape != kmax.shape or kmin.shape[0] != batch or kmin.shape[3] != head_dim:
        raise ConfigError(f"quest bounds {tuple(kmin.shape)} / {tuple(kmax.shape)} do not match the query")
    kv_heads = kmin.shape[1]
    if q_heads % kv_heads:
        raise ConfigError(f"{q_heads} query heads are not a multiple of {kv_heads} KV heads")
    if kmin.dtype != torch.bfloat16 or kmax.dtype != torch.bfloat16 or kmin.stride() != kmax.stride():
        raise ConfigError("quest bounds must be bf16 tensors of equal strides")
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
        "eco_quest_select", query.data_ptr(), query.stride(0), query.stride(2), query.stride(1), kmin.data_ptr(),
        kmax.data_ptr(), kmin.stride(0), kmin.stride(1), kmin.stride(2), done.data_ptr(), max_done, pages,
        int(bool(first_page)), out.data_ptr(), batch, queries, q_heads, kv_heads, head_dim, scores.data_ptr(), scores.numel() * 4,
        _lib.stream_of(device),
    )
    return out


@dataclass
class QuestPages:
    """Page bounds of one layer's committed cache (the reference's ``QuestPages``, attention/quest.py:112-204).

    Attributes:
        kmin: bf16 ``[B, Hkv, P, D]`` channel-wise smallest key of every committed page.
        kmax: bf16 ``[B, Hkv, P, D]`` the largest keys.
        done: int32 ``[B]`` committed pages of every row; tokens from ``done[b] * page`` on are read densely.
        min_done: ``min(done)``, on the host.
        max_done: ``max(done)``, on the host.
        page: Tokens per Quest page (a power of two, at least 16).
        pages: Committed pages every row and KV head reads.
        max_queries: Longest query that is restricted to the pages; longer ones see every key.
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
    first_page: bool = False
    format: str = "quest"

    def select(self, query: torch.Tensor) -> torch.Tensor:
        """int32 ``[B, Hkv, pages]`` selected pages for ``query`` ``[B, Hq, Q, D]`` (see :func:`select_pages`)."""
        return select_pages(query, self.kmin, self.kmax, self.done, self.max_done, self.pages, self.first_page)

    def attend(self, query: torch.Tensor, cache: PagedKVCache, block_table: torch.Tensor, seq_lens: torch.Tensor,
               max_seq_len: int, scale: float | None = None, softcap: float | None = None,
               sinks: torch.Tensor | None = None, mask: torch.Tensor | None = None) -> torch.Tensor:
        """``[B, Q, Hq, D]`` attention of ``query`` ``[B, Hq, Q, D]`` over the selected pages and the dense tail; a
        query longer than :attr:`max_queries` attends densely (attention/quest.py:191-204)."""
        if query.shape[2] > self.max_queries:
            return paged_decode_attention(query.transpose(1, 2), cache, block_table, seq_lens, max_seq_len, scale,
                                          softcap, sinks, mask=mask)
        return quest_decode_attention(query, cache, block_table, seq_lens, max_seq_len, self, scale, softcap, sinks,
                                      mask=mask)


def quest_decode_attention(query: torch.Tensor, cache: PagedKVCache, block_table: torch.Tensor,
                           seq_lens: torch.Tensor, max_seq_len: int, pages: QuestPages, scale: float | None = None,
                           softcap: float | None = None, sinks: torch.Tensor | None = None,
                           out: torch.Tensor | None = None, index: torch.Tensor | None = None,
                           mask: torch.Tensor | None = None) -> torch.Tensor:
    """Paged decode attention over the selected pages and the dense tail (attention/quest.py:239-344).

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
    _check_page(pages.page)
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
    :meth:`pages` hands the selection and the attention ``max_done = max_pages``: the calls of a decode step then
    have fixed shapes and no host value that changes from step to step. Pages past a row's ``done`` score ``-inf``,
    so the selection equals the one with the batch's true ``max(done)`` whenever it exceeds ``pages``; a row with at
    most ``pages`` committed pages selects all of them (dense attention, in another key order).
    """

    def __init__(self, batch: int, kv_heads: int, head_dim: int, max_pages: int, page: int, pages: int,
                 device: torch.device | str, max_queries: int = 1, first_page: bool = False) -> None:
        _check_page(page)
        if max_pages <= 0 or pages <= 0:
            raise ConfigError(f"quest state needs positive max_pages and pages, got {max_pages}, {pages}")
        shape = (batch, kv_heads, max_pages, head_dim)
        self.kmin = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.kmax = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        self.valid = torch.zeros(batch * kv_heads, dtype=torch.int32, device=device)
        self.done = torch.zeros(batch, dtype=torch.int32, device=device)
        self.page, self.pages, self.max_pages, self.max_queries = page, pages, max_pages, max_queries
        self.first_page = first_page

    def reset(self) -> None:
        """Forget every page (a new generation in the same buffers)."""
        self.valid.zero_()
        self.done.zero_()

    def refresh(self, cache: PagedKVCache, block_table: torch.Tensor, committed: torch.Tensor) -> None:
        """Bounds of the pages below ``committed`` (int32 ``[B]`` tokens, on the device) not computed yet; ``done``
        becomes ``committed // page`` (at most ``max_pages``)."""
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
        _lib.call(
            "eco_quest_refresh_bounds", cache.keys.data_ptr(), _lib.fmt(cache.dtype), cache.num_pages,
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1], committed.data_ptr(),
            self.valid.data_ptr(), self.done.data_ptr(), self.page, self.kmin.data_ptr(), self.kmax.data_ptr(),
            self.kmin.stride(0), self.kmin.stride(1), self.kmin.stride(2), self.max_pages, batch, cache.kv_heads,
            cache.head_dim, PAGE, _lib.stream_of(device),
        )

    def pages_handle(self) -> QuestPages:
        """The layer's :class:`QuestPages` with the device ``done`` and ``max_done = max_pages``."""
        return QuestPages(self.kmin, self.kmax, self.done, 0, self.max_pages, self.page, self.pages,
                          self.max_queries, self.first_page)
