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
    """One layer's prompt after an eviction kept part of it: the attachment of format ``"gathered"`` that
    :func:`gathered_decode_attention` reads (the reference's GatheredKV fields, attention/gathered.py:39-64).

    Attributes:
        key: ``[B, Hkv, C, D]``: row ``b`` and KV head ``h`` keep their surviving prompt keys in the first
            ``count[b, h]`` entries, in slot order; the entries past the count are never read.
        value: ``[B, Hkv, C, Dv]``: the values of those entries.
        index: int32 ``[B, Hkv, C]``: the slot each kept entry came from, which is the mask column it is read with.
        count: int32 ``[B, Hkv]``: how many entries each row and KV head kept.
        start: int32 ``[B]``: the first slot of row ``b`` read from the dense buffers (the end of its prompt).
        dropped: The smallest ``start[b] - count[b, h]`` over the batch, a host int: the virtual key axis of a call is
            ``S - dropped`` keys long.
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


def _validate(g: GatheredKV, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
    """What ``eco_gathered_decode`` needs of the attachment, checked before the launch: the compact entries share the
    dense buffers' rows, heads, channels, dtype and device and have unit channel strides; the slot index has unit
    stride along the entries; the counts and starts are dense int32 vectors the kernel addresses as ``b * Hkv + h``
    and ``b``; ``dropped`` lies within the slots."""
    batch, kv_heads, slots = key.shape[:3]
    entries = g.key.shape[2] if g.key.dim() == 4 else -1
    for what, compact, dense in (("keys", g.key, key), ("values", g.value, value)):
        if compact.dim() != 4 or tuple(compact.shape) != (batch, kv_heads, entries, dense.shape[3]):
            raise ConfigError(f"the gathered {what} {tuple(compact.shape)} do not fit the cache's "
                              f"{tuple(dense.shape)} ({entries} kept entries)")
        if compact.dtype != dense.dtype or compact.device != query.device or compact.stride(3) != 1:
            raise ConfigError(f"the gathered {what} must be {dense.dtype} on {query.device} with unit channel stride")
    if g.index.dtype != torch.int32 or tuple(g.index.shape) != (batch, kv_heads, entries) or \
            g.index.device != query.device or g.index.stride(2) != 1:
        raise ConfigError(f"the gathered slot index must be int32 [{batch}, {kv_heads}, {entries}] with unit stride "
                          f"along the entries on {query.device}")
    for what, t, shape in (("counts", g.count, (batch, kv_heads)), ("starts", g.start, (batch,))):
        if t.dtype != torch.int32 or tuple(t.shape) != shape or not t.is_contiguous() or t.device != query.device:
            raise ConfigError(f"the gathered {what} must be a contiguous int32 {list(shape)} on {query.device}")
    if not 0 <= g.dropped <= slots:
        raise ConfigError(f"a gathered cache of {slots} slots cannot drop {g.dropped} of them")


def gathered_decode_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
                              scale: float, gathered: GatheredKV, softcap: float | None = None,
                              out: torch.Tensor | None = None, sinks: torch.Tensor | None = None,
                              launch: object = None) -> torch.Tensor:
    """Attention of a few queries per row over the kept prompt entries followed by the dense slots from ``start[b]``
    on: the reference's gathered_decode_attention (attention/gathered.py:96-179) on ``eco_gathered_decode``.

    Args:
        query: ``[B, Hq, Q, D]``; bf16, fp16 or fp32.
        key: ``[B, Hkv, S, D]`` dense keys in the query's dtype; the kernel reads only their slots from ``start[b]`` on.
        value: ``[B, Hkv, S, Dv]`` dense values, read the same way.
        mask: ``None``, or a boolean ``[B, 1 or Hq, Q, S]`` over the original slots (a kept entry reads the column of
            the slot it came from).
        scale: The score multiplier.
        gathered: The kept prompt entries.
        softcap: Optional tanh soft cap on the scaled scores.
        out: Optional ``[B, Q, Hq, Dv]`` destination.
        sinks: Optional ``[Hq]`` sink logits in the softmax denominator.
        launch: Accepted for the reference's signature; the launch plan here follows from the shapes alone.

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
    _validate(gathered, query, key, value)
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
        raise ConfigError(f"gathered_decode_attention supports head dims up to 512, got {head_dim} / {head_dv}")
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
