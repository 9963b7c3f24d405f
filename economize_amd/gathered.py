"""Decode attention over a physically compacted KV cache on the GPU (the reference's attention/gathered.py:1-179).

A prompt-time eviction (SnapKV, H2O as KVCache-Factory runs them) keeps a subset of the prompt entries of every
row and KV head; :class:`GatheredKV` holds those entries contiguously, and :func:`gathered_decode_attention` reads
them followed by the dense slots from ``start[b]`` on, through the dense decode kernel's virtual key axis
(``eco_gathered_decode``): for row ``b`` and KV head ``h`` the first ``count[b, h]`` virtual keys are the compact
entries (their original slots ``index`` are their mask columns, so causal, tree and sliding-window masks apply
unchanged), and virtual key ``count[b, h] + i`` is dense slot ``start[b] + i``. The result is the dense attention
with the evicted entries masked, summed in another order.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .decode import DOT_DTYPES, _channel_contiguous, _workspace, mask_operand, sinks_operand
from .errors import ConfigError

__all__ = ["GatheredKV", "gathered_decode_attention"]


@dataclass
class GatheredKV:
    """Compacted prompt entries of one layer (a packed K/V of format ``"gathered"``, attention/gathered.py:39-64).

    Attributes:
        key: ``[B, Hkv, C, D]`` kept prompt keys of every row and KV head, in slot order (``C >= count[b, h]``).
        value: ``[B, Hkv, C, Dv]`` the matching values.
        index: int32 ``[B, Hkv, C]`` original slot of every compact entry (its mask column).
        count: int32 ``[B, Hkv]`` compact entries of every row and KV head.
        start: int32 ``[B]`` first dense slot read for row ``b``.
        dropped: ``min(start[b] - count[b, h])``, on the host: the virtual key axis is ``keys - dropped`` long.
    """

    key: torch.Tensor
    value: torch.Tensor
    index: torch.Tensor
    count: torch.Tensor
    start: torch.Tensor
    dropped: int
    format: str = "gathered"

    def attend(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
               scale: float, softcap: float | None = None, sinks: torch.Tensor | None = None) -> torch.Tensor:
        return gathered_decode_attention(query, key, value, mask, scale, self, softcap=softcap, sinks=sinks)


def _check(g: GatheredKV, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
    """The reference's layout checks (attention/gathered.py:67-93)."""
    batch, kv_heads = key.shape[:2]
    capacity = g.key.shape[2]
    expected = {
        "key": ((batch, kv_heads, capacity, key.shape[3]), key.dtype),
        "value": ((batch, kv_heads, capacity, value.shape[3]), value.dtype),
        "index": ((batch, kv_heads, capacity), torch.int32),
        "count": ((batch, kv_heads), torch.int32),
        "start": ((batch,), torch.int32),
    }
    for name, (shape, dtype) in expected.items():
        t = getattr(g, name)
        if tuple(t.shape) != shape or t.dtype != dtype or t.device != query.device:
            raise ConfigError(f"gathered {name} is {tuple(t.shape)} {t.dtype} on {t.device}, expected {shape} {dtype} "
                              f"on {query.device}")
        if (t.stride(-1) != 1) if name in ("key", "value") else not t.is_contiguous():
            raise ConfigError(f"gathered {name} is not laid out for the kernel (strides {t.stride()})")
    if g.dropped < 0 or g.dropped > key.shape[2]:
        raise ConfigError(f"gathered cache drops {g.dropped} of {key.shape[2]} slots")


def gathered_decode_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
                              scale: float, gathered: GatheredKV, softcap: float | None = None,
                              out: torch.Tensor | None = None, sinks: torch.Tensor | None = None,
                              launch: object = None) -> torch.Tensor:
    """Decode attention over the compact entries and the dense tail (attention/gathered.py:96-179).

    Args:
        query: ``[B, Hq, Q, D]``, bf16, fp16 or fp32.
        key: Dense ``[B, Hkv, S, D]`` in the query's dtype; read only at slots ``>= gathered.start[b]``.
        value: Dense ``[B, Hkv, S, Dv]``; likewise.
        mask: Boolean ``[B, 1 or Hq, Q, S]`` over the original slots, or ``None``.
        scale: Multiplier of the scores.
        gathered: The compact entries.
        softcap: Optional tanh soft cap of the scaled scores.
        out: Optional ``[B, Q, Hq, Dv]`` output buffer.
        sinks: Optional ``[Hq]`` attention-sink logits.
        launch: The reference's launch override; the plan here is a function of the shapes, so it is ignored.

    Returns:
        ``[B, Q, Hq, Dv]`` in the query's dtype.
    """
    del launch
    device = _lib.require_gpu(query, key, value, gathered.key)
    batch, q_heads, queries, head_dim = query.shape
    _, kv_heads, keys, _ = key.shape
    head_dv = value.shape[-1]
    if q_heads % kv_heads:
        raise ConfigError(f"{q_heads} query heads are not a multiple of {kv_heads} KV heads")
    if query.dtype not in DOT_DTYPES or key.dtype != query.dtype or value.dtype != query.dtype:
        raise ConfigError(f"gathered_decode_attention takes K/V in the query's dtype, got {key.dtype} / {value.dtype}")
    if keys == 0:
        raise ConfigError("gathered_decode_attention needs a cache of at least one slot")
    _check(gathered, query, key, value)
    m, mask_strides = mask_operand(mask, keys)
    sinks = sinks_operand(sinks, q_heads)
    if out is not None and (out.shape != (batch, queries, q_heads, head_dv) or out.dtype != query.dtype or
                            out.stride(-1) != 1):
        raise ConfigError("out must be [B, Q, Hq, Dv] in the query's dtype with a contiguous last axis")
    query, key, value = _channel_contiguous(query), _channel_contiguous(key), _channel_contiguous(value)
    ck, cv = _channel_contiguous(gathered.key), _channel_contiguous(gathered.value)
    if out is None:
        out = torch.empty(batch, queries, q_heads, head_dv, dtype=query.dtype, device=device)
    virtual = max(1, keys - gathered.dropped)
    need = int(_lib.lib().eco_decode_workspace_size(batch, queries, q_heads, kv_heads, virtual, head_dim, head_dv))
    if need == 0:
        raise ConfigError(f"gathered_decode_attention supports head dims up to 256, got {head_dim} / {head_dv}")
    ws = _workspace(need, device, batch, queries, q_heads, kv_heads)
    idx = gathered.index
    _lib.call(
        "eco_gathered_decode", query.data_ptr(), _lib.fmt(query.dtype), query.stride(0), query.stride(1),
        query.stride(2), key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), key.stride(2),
        value.stride(0), value.stride(1), value.stride(2), ck.data_ptr(), cv.data_ptr(), ck.stride(0), ck.stride(1),
        ck.stride(2), cv.stride(0), cv.stride(1), cv.stride(2), idx.data_ptr(), idx.stride(0), idx.stride(1),
        gathered.count.data_ptr(), gathered.start.data_ptr(), ck.shape[2], int(gathered.dropped), _lib.ptr(m),
        *mask_strides, _lib.ptr(sinks), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), batch, queries,
        q_heads, kv_heads, keys, head_dim, head_dv, float(scale if scale is not None else 1 / math.sqrt(head_dim)),
        float(softcap or 0.0), ws.data_ptr(), ws.numel(), _lib.stream_of(device),
    )
    return out
