"""Decode attention over compacted prompt entries (oracle).

Restates the virtual key axis of attention/gathered.py:1-14 and _gathered_kernels.py:13-123 of the reference: for row
``b`` and KV head ``h``, virtual key ``t < count[b, h]`` is compact entry ``t`` (keys ``ck``, values ``cv``) whose mask
column is its original slot ``index[b, h, t]``; virtual key ``count[b, h] + i`` is dense slot ``start[b] + i`` with
mask column ``start[b] + i``. The attention over that axis is :func:`oracle.attention.reference_attention` of the
virtual K/V with a virtual mask (positions past a row's axis hidden).

Pinned by (``tests/test_oracle_gathered.py``): when the compact entries are the kept dense entries themselves, the
result equals ``reference_attention`` over the whole dense cache with the evicted prompt entries masked, the
reference's own statement of what the kernel computes (gathered.py:12-14); closed forms for no compact entry
(``start = 0``: dense attention) and no dense tail.
"""

from __future__ import annotations

import numpy as np

from .attention import reference_attention

__all__ = ["gathered_reference"]


def gathered_reference(query: np.ndarray, key: np.ndarray, value: np.ndarray, mask: np.ndarray | None, scale: float,
                       ck: np.ndarray, cv: np.ndarray, index: np.ndarray, count: np.ndarray, start: np.ndarray,
                       softcap: float | None = None, sinks: np.ndarray | None = None) -> np.ndarray:
    """``[B, Q, Hq, Dv]`` float32: ``query`` ``[B, Hq, Q, D]`` over the virtual axis of compact entries
    ``ck`` / ``cv`` ``[B, Hkv, C, D / Dv]`` then dense slots of ``key`` / ``value`` ``[B, Hkv, S, D / Dv]`` from
    ``start[b]`` on; ``mask`` boolean ``[B or 1, 1 or Hq, Q or 1, S]`` over the original slots."""
    q = np.asarray(query, dtype=np.float32)
    batch, q_heads, queries, _ = q.shape
    kv_heads, slots = key.shape[1], key.shape[2]
    groups = q_heads // kv_heads
    out = np.zeros((batch, queries, q_heads, value.shape[3]), np.float32)
    for b in range(batch):
        for h in range(kv_heads):
            c, s0 = int(count[b, h]), int(start[b])
            cols = np.concatenate([np.asarray(index[b, h, :c], np.int64), np.arange(s0, slots)])
            vk = np.concatenate([ck[b, h, :c], key[b, h, s0:]], axis=0)[None, None]
            vv = np.concatenate([cv[b, h, :c], value[b, h, s0:]], axis=0)[None, None]
            heads = slice(h * groups, (h + 1) * groups)
            vm = None
            if mask is not None:
                full = np.broadcast_to(mask, (batch, q_heads, queries, slots))
                vm = full[b: b + 1, heads][..., cols]
            sk = None if sinks is None else np.asarray(sinks, np.float32)[heads]
            out[b, :, heads] = reference_attention(q[b: b + 1, heads], vk, vv, vm, scale, softcap, sk)[0]
    return out
