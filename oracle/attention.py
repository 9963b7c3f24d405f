"""The fp32 attention definition (oracle).

``reference_attention`` restates attention/decode.py:66-103 of the reference: grouped-query heads repeated over
their group (``repeat_interleave``), ``scores = q @ k^T * scale`` in fp32, the optional ``softcap * tanh(s / softcap)``,
hidden keys at ``-inf``, the optional attention-sink logit in the denominator, softmax, NaN (a row that sees nothing)
to 0, ``probs @ v``, output transposed to ``[B, Q, Hq, Dv]``.

Pinned by (``tests/test_oracle_attention.py``): brute-force loops over tiny inputs (one exp per key, no matrix
products), the closed forms of a single visible key (output = that key's value), uniform scores (output = mean of
the visible values), a row that sees nothing (exact 0) and the sink identity (a sink at -inf changes nothing), and
invariance of GQA under repeating the KV heads.
"""

from __future__ import annotations

import numpy as np

__all__ = ["reference_attention"]


def reference_attention(query: np.ndarray, key: np.ndarray, value: np.ndarray, mask: np.ndarray | None,
                        scale: float, softcap: float | None = None, sinks: np.ndarray | None = None) -> np.ndarray:
    """``[B, Q, Hq, Dv]`` float32 attention of ``query`` ``[B, Hq, Q, D]`` over ``key`` ``[B, Hkv, S, D]`` and
    ``value`` ``[B, Hkv, S, Dv]`` (decode.py:66-103). ``mask`` is boolean ``[B or 1, 1 or Hq, Q or 1, S]``
    (True = visible) or None."""
    q = np.asarray(query, dtype=np.float32)
    groups = q.shape[1] // key.shape[1]
    k = np.repeat(np.asarray(key, dtype=np.float32), groups, axis=1)
    v = np.repeat(np.asarray(value, dtype=np.float32), groups, axis=1)
    scores = np.matmul(q, np.swapaxes(k, -1, -2)).astype(np.float32) * np.float32(scale)
    if softcap is not None:
        c = np.float32(softcap)
        scores = (c * np.tanh(scores / c)).astype(np.float32)
    if mask is not None:
        scores = np.where(np.broadcast_to(mask, scores.shape), scores, -np.inf).astype(np.float32)
    if sinks is not None:
        sink = np.broadcast_to(np.asarray(sinks, dtype=np.float32).reshape(1, -1, 1, 1), (*scores.shape[:3], 1))
        full = np.concatenate([scores, sink], axis=-1)
        m = full.max(axis=-1, keepdims=True)
        e = np.exp(full - m)
        probs = (e / e.sum(axis=-1, keepdims=True))[..., :-1]
    else:
        m = scores.max(axis=-1, keepdims=True)
        with np.errstate(invalid="ignore"):
            e = np.exp(scores - np.where(np.isfinite(m), m, 0))
            probs = e / e.sum(axis=-1, keepdims=True)
        probs = np.nan_to_num(probs, nan=0.0)
    out = np.matmul(probs.astype(np.float32), v).astype(np.float32)
    return np.swapaxes(out, 1, 2)
