"""KIVI on vLLM's paged cell layout, on the GPU (the reference's backends/vllm/kivi/layout.py and kernels.py).

vLLM keeps one *cell* per (page, KV head, token) of every attention layer; KIVI's cell holds the token's dense K/V
(vLLM's own kernels and the full-precision residual read them) followed by what its packed form needs::

    [ K: D elements | V: D elements | value scales: nvg fp16 | value zeros: nvg fp16 |
      key aux: ka fp16 | key codes: D/pb bytes | value codes: D/pb bytes | key flag | value flag ]  (16-byte aligned)

:func:`quantize_committed` quantizes, before a pass attends, the keys below ``(c // R) * R`` and the values below
``c - R`` of every decoding request (``c`` = the tokens the cache held before the pass), newest first, until a cell
already quantized (``eco_kivi_cells_quantize``), leaving every cell as the reference's ``write_cells`` lays it out; a
quantized cell's dense entry holds the dequantized value, so attention over the dense entries is attention over the
KIVI numbers. :func:`clear_flags` marks cells vLLM's cache write just filled as full precision.
:func:`paged_kivi_attention` is the reference's attention over the cells with vLLM's varlen query layout and a
causal bound per query (kernels.py:216-415): the dense decode kernel reading the cells through the block table
(``eco_kivi_cells_attention``). As the reference's kernel does (kernels.py:274-296), a key or value whose cell flag is
1 is read through its codes, scales and zero points, and its dense entry is ignored, for bf16 cells of 128 channels
with key groups of 32, 2- or 4-bit codes and pages of a multiple of 32 tokens; every other cell (flag 0 or 2), every
other cell shape, and every cell when the environment sets ``ECO_CELLS_DENSE=1``, is read from its dense entry, which
quantize_committed left holding the same dequantized number.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib
from .errors import ConfigError

__all__ = ["FLAG_DENSE", "FLAG_OVERFLOW", "FLAG_PACKED", "CellLayout", "cache_views", "cell_layout", "clear_flags",
           "paged_kivi_attention", "quantize_committed"]

FLAG_DENSE, FLAG_PACKED, FLAG_OVERFLOW = 0, 1, 2
_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


@dataclass(frozen=True)
class CellLayout:
    """Byte offsets inside one cell (layout.py:133-193)."""

    head_size: int
    element_size: int
    bits: int
    group_size: int
    value_group: int
    key_aux: int
    off_v: int
    off_vs: int
    off_vz: int
    off_ka: int
    off_kc: int
    off_vc: int
    off_flag: int
    size: int

    @property
    def value_groups(self) -> int:
        return self.head_size // self.value_group

    @property
    def dense_size(self) -> int:
        """Bytes of the cell without KIVI (vLLM's ``2 * head_size`` elements)."""
        return self.off_vs


def cell_layout(head_size: int, dtype: torch.dtype, bits: int, group_size: int) -> CellLayout:
    """The cell of a layer with ``head_size`` channels in ``dtype`` (layout.py:196-213).

    Raises:
        ConfigError: A head size (a power of two from 16 to 256), bits (2, 4, 8) or group (a power of two up to 128)
            the packing does not take.
    """
    if dtype not in _DTYPES:
        raise ConfigError(f"KIVI cells hold bf16, fp16 or fp32 entries, not {dtype}")
    es = torch.empty((), dtype=dtype).element_size()
    out = (ctypes.c_int32 * 10)()
    _lib.call("eco_kivi_cells_layout", head_size, es, bits, group_size, ctypes.addressof(out))
    return CellLayout(head_size, es, bits, group_size, *out)


def cache_views(kv_cache: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The typed and byte views of one layer's cache ``[pages, heads, page_size, cell elements]`` (kernels.py:
    44-55)."""
    if kv_cache.dim() != 4 or kv_cache.stride(-1) != 1:
        raise ConfigError(f"KIVI cells need a [pages, heads, tokens, cell] cache with a contiguous cell, got shape "
                          f"{tuple(kv_cache.shape)} strides {kv_cache.stride()}")
    return kv_cache, kv_cache.view(torch.uint8)


def _cells_args(kv_cache: torch.Tensor, layout: CellLayout) -> list:
    typed, u8 = cache_views(kv_cache)
    if typed.dtype not in _DTYPES or typed.element_size() != layout.element_size:
        raise ConfigError(f"the cache dtype {typed.dtype} is not the layout's ({layout.element_size}-byte entries)")
    if u8.shape[3] < layout.size:
        raise ConfigError(f"cells of {u8.shape[3]} bytes do not hold the layout's {layout.size}")
    return [u8.data_ptr(), _lib.fmt(typed.dtype), u8.stride(0), u8.stride(1), u8.stride(2), u8.shape[0], u8.shape[2],
            u8.shape[1]]


def quantize_committed(kv_cache: torch.Tensor, layout: CellLayout, residual_length: int, block_table: torch.Tensor,
                       query_start_loc: torch.Tensor, seq_lens: torch.Tensor, prefilling: torch.Tensor) -> None:
    """Quantize the committed tokens that left the residual of every decoding request (kernels.py:180-207).

    Args:
        kv_cache: One layer's cache, typed ``[pages, heads, page_size, cell elements]``.
        layout: Its cell layout.
        residual_length: ``R`` (whole key groups).
        block_table: int32 ``[requests, pages per request]``.
        query_start_loc: int32 ``[requests + 1]``, vLLM's varlen query offsets.
        seq_lens: int32 ``[requests]``, tokens of each request after the pass.
        prefilling: int32 ``[requests]``, nonzero for a request whose prompt is not done.
    """
    device = _lib.require_gpu(kv_cache, block_table, query_start_loc, seq_lens, prefilling)
    args = _cells_args(kv_cache, layout)
    requests = seq_lens.shape[0]
    for name, t, n in (("query_start_loc", query_start_loc, requests + 1), ("seq_lens", seq_lens, requests),
                       ("prefilling", prefilling, requests)):
        if t.dtype != torch.int32 or t.shape != (n,) or not t.is_contiguous():
            raise ConfigError(f"{name} must be a contiguous int32 [{n}]")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1 or \
            block_table.shape[0] < requests:
        raise ConfigError("block_table must be int32 [requests, pages] with contiguous rows")
    if args[6] % layout.group_size:
        raise ConfigError(f"KIVI needs pages of whole key groups: {args[6]} tokens per page, groups of "
                          f"{layout.group_size}")
    # the walk's stopping points per (request, KV head), found before any cell changes
    plan = torch.empty(4 * requests * args[7], dtype=torch.int32, device=device)
    _lib.call("eco_kivi_cells_quantize", *args, block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
              query_start_loc.data_ptr(), seq_lens.data_ptr(), prefilling.data_ptr(), requests, layout.head_size,
              layout.bits, layout.group_size, residual_length, plan.data_ptr(), _lib.stream_of(device))


def clear_flags(kv_cache: torch.Tensor, slot_mapping: torch.Tensor, layout: CellLayout) -> None:
    """Mark the cells of ``slot_mapping`` (int32, ``page * page_size + position``; negative slots are padding) as
    full precision (kernels.py:58-78)."""
    device = _lib.require_gpu(kv_cache, slot_mapping)
    if slot_mapping.dtype != torch.int32 or slot_mapping.dim() != 1 or not slot_mapping.is_contiguous():
        raise ConfigError("slot_mapping must be a contiguous int32 [tokens]")
    _lib.call("eco_kivi_cells_clear_flags", *_cells_args(kv_cache, layout), slot_mapping.data_ptr(),
              slot_mapping.shape[0], layout.head_size, layout.bits, layout.group_size, _lib.stream_of(device))


def paged_kivi_attention(query: torch.Tensor, kv_cache: torch.Tensor, layout: CellLayout, block_table: torch.Tensor,
                         query_start_loc: torch.Tensor, seq_lens: torch.Tensor, max_query_len: int, keys: int,
                         scale: float | None = None, out: torch.Tensor | None = None, softcap: float | None = None,
                         sinks: torch.Tensor | None = None) -> torch.Tensor:
    """Attention of vLLM's varlen queries over the cells (kernels.py:354-415).

    Args:
        query: ``[tokens, Hq, D]`` in the cache dtype (channel stride 1); request ``b``'s queries are tokens
            ``query_start_loc[b] .. query_start_loc[b + 1] - 1``.
        kv_cache: One layer's cache, typed ``[pages, heads, page_size, cell elements]``.
        layout: Its cell layout.
        block_table: int32 ``[requests, pages per request]``.
        query_start_loc: int32 ``[requests + 1]``.
        seq_lens: int32 ``[requests]``: query ``i`` of a request of ``n`` queries sees keys ``< seq_len - n + i + 1``.
        max_query_len: The longest query of the batch.
        keys: The longest ``seq_len`` of the batch.
        scale: Multiplier of the scores (``1 / sqrt(D)`` by default).
        out: Optional ``[tokens, Hq, D]`` output in the query's dtype.
        softcap: Optional tanh soft cap.
        sinks: Optional ``[Hq]`` attention-sink logits.

    Returns:
        ``[tokens, Hq, D]``.
    """
    device = _lib.require_gpu(query, kv_cache, block_table, query_start_loc, seq_lens)
    typed, u8 = cache_views(kv_cache)
    if query.dim() != 3 or query.dtype != typed.dtype or query.stride(-1) != 1:
        raise ConfigError("paged_kivi_attention takes queries [tokens, Hq, D] in the cache dtype with contiguous "
                          "channels")
    tokens, q_heads, dim = query.shape
    requests = seq_lens.shape[0]
    if dim != layout.head_size:
        raise ConfigError(f"queries of {dim} channels for cells of {layout.head_size}")
    for name, t, n in (("query_start_loc", query_start_loc, requests + 1), ("seq_lens", seq_lens, requests)):
        if t.dtype != torch.int32 or t.shape != (n,) or not t.is_contiguous():
            raise ConfigError(f"{name} must be a contiguous int32 [{n}]")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ConfigError("block_table must be int32 [requests, pages] with contiguous rows")
    if block_table.shape[0] < requests:
        raise ConfigError(f"block_table has {block_table.shape[0]} rows for {requests} requests")
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or out.stride(-1) != 1:
        raise ConfigError("out must be [tokens, Hq, D] in the query's dtype with contiguous channels")
    if requests == 0 or tokens == 0:
        return out
    s = None
    if sinks is not None:
        if sinks.numel() != q_heads:
            raise ConfigError(f"{sinks.numel()} sink logits for {q_heads} query heads")
        s = sinks.reshape(-1).float().contiguous()
    need = int(_lib.lib().eco_kivi_cells_attention_workspace_size(requests, max_query_len, q_heads, u8.shape[1],
                                                                   max(keys, 1), dim))
    if need == 0:
        raise ConfigError("paged_kivi_attention: unsupported shape")
    from .decode import _workspace

    ws = _workspace(need, device, requests, int(max_query_len), q_heads, u8.shape[1])
    scale = 1.0 / math.sqrt(dim) if scale is None else scale
    _lib.call("eco_kivi_cells_attention", query.data_ptr(), query.stride(0), query.stride(1), u8.data_ptr(),
              _lib.fmt(typed.dtype), u8.stride(0), u8.stride(1), u8.stride(2), u8.shape[0], u8.shape[2], u8.shape[1],
              block_table.data_ptr(), block_table.stride(0), block_table.shape[1], query_start_loc.data_ptr(),
              seq_lens.data_ptr(), requests, int(max_query_len), max(int(keys), 1), dim, layout.bits,
              layout.group_size, _lib.ptr(s), out.data_ptr(), out.stride(0), out.stride(1), q_heads, float(scale),
              float(softcap or 0.0), ws.data_ptr(), ws.numel(), _lib.stream_of(device))
    return out
