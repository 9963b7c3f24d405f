"""Quest page bounds, page selection and the restricted attention (oracle).

Follows attention/quest.py of the reference:

* ``page_bounds`` (quest.py:54-65): channel-wise min and max of every page's keys (fp8 keys exact in bf16).
* ``select_pages`` (quest.py:73-108): ``qsum`` / ``qabs`` = sums of ``q`` / ``|q|`` over the group's heads and the
  pass's queries; ``score = sum_d qsum_d * (lo_d + hi_d) * 0.5 + sum_d qabs_d * (hi_d - lo_d) * 0.5`` (two dot
  products, then their sum); pages at or past ``done[b]`` score ``-inf``; the top ``min(pages, max_done)`` indices,
  those past ``done[b]`` dropped, sorted ascending and padded with ``-1``.
* ``keep`` / ``restrict_mask`` (quest.py:145-189) and ``quest_reference`` (quest.py:207-219): the selected pages plus
  every slot from ``done[b] * page`` on, attended with the fp32 definition.
* the virtual key axis of ``_quest_split_kernel`` (attention/_quest_kernels.py:55-87): the selected pages in slot
  order, then the dense tail.

Two choices the reference leaves open are fixed here, and the HIP kernels make the same ones:

* the fp32 summation order of the two dot products (torch's einsum order is unspecified): per page, products
  ``a_d * b_d`` rounded to fp32; sequential sums over runs of 8 channels; then a halving tree over the runs (run
  ``j`` plus run ``j + n/2``), ``n`` padded to a power of two with zeros. ``qsum``/``qabs`` add the rows in order
  ``r = g * Q + q``.
* ties of ``torch.topk`` (unspecified order): equal scores are taken lowest page index first.

Pinned by (``tests/test_oracle_quest.py``): a float64 computation of the per-head bound ``sum_h sum_d max(q_hd lo_d,
q_hd hi_d)`` (the mathematically equal form of the official Quest selection, tests/techniques/test_quest.py:124-143
describes it) selects the same pages whenever the gap at the k-th score exceeds the fp32 error bound; brute-force
page masks for ``keep``; the invariants of test_quest.py:202-215 (increasing order, ``-1`` padding, every committed
page when ``done <= pages``). End to end, ``tests/test_golden_reference.py`` decodes the reference's golden model
with :func:`page_bounds`, :func:`select_pages` and :func:`quest_reference` and gets the reference's own ``kv_quest``
golden tokens (tests/golden/catalog.py:195-207). The reference's own ``select_pages``, run on the CPU, wrote the
selections of ``tests/golden/quest_select_vectors.npz`` (``tests/test_oracle_quest_vectors.py``): random keys at
head dims 64 / 128, fp8 keys, four query rows, a planted workload and short rows select exactly its pages. Two cases
differ by what the definition leaves open: exact ties, where torch's CPU ``topk`` keeps higher-index members of a
tied group (same scores selected, lower index here), and near ties of about one fp32 unit, where torch's CPU einsum
rounds 127 of 320 scores differently from the fixed order above (every page the selections disagree on lies within
the fp32 error bound of the k-th score). The exact fp32 score bits at such near ties are parity unpinned: the
reference's own bits there follow its backend's einsum order (CPU and GPU differ), so no check can fix them.
"""

from __future__ import annotations

import numpy as np

from .attention import reference_attention

__all__ = ["keep_slots", "page_bounds", "page_scores", "quest_reference", "select_pages", "tree_dot"]


def page_bounds(keys: np.ndarray, first: int, last: int, page: int) -> tuple[np.ndarray, np.ndarray]:
    """``(kmin, kmax)`` ``[B, H, last - first, D]`` of pages ``first .. last - 1`` of ``keys`` ``[B, H, S, D]``
    (float32 holding the key values; quest.py:54-65)."""
    block = np.asarray(keys[:, :, first * page: last * page], dtype=np.float32)
    b, h, _, d = block.shape
    block = block.reshape(b, h, last - first, page, d)
    return block.min(axis=3), block.max(axis=3)


def tree_dot(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """``sum_d a_d * b_d`` over the last axis in the canonical fp32 order (see the module docstring)."""
    prod = (np.asarray(a, dtype=np.float32) * np.asarray(b, dtype=np.float32)).astype(np.float32)
    d = prod.shape[-1]
    runs = -(-d // 8)
    n = 1 << max(0, runs - 1).bit_length()
    pad = n * 8 - d
    if pad:
        prod = np.concatenate([prod, np.zeros((*prod.shape[:-1], pad), np.float32)], axis=-1)
    chunks = prod.reshape(*prod.shape[:-1], n, 8)
    t = chunks[..., 0]
    for i in range(1, 8):
        t = (t + chunks[..., i]).astype(np.float32)
    while n > 1:
        n //= 2
        t = (t[..., :n] + t[..., n:]).astype(np.float32)
    return t[..., 0]


def query_sums(query: np.ndarray, kv_heads: int) -> tuple[np.ndarray, np.ndarray]:
    """``(qsum, qabs)`` ``[B, Hkv, D]``: the group's rows ``r = g * Q + q`` added in order (quest.py:93-95)."""
    q = np.asarray(query, dtype=np.float32)
    b, hq, nq, d = q.shape
    rows = q.reshape(b, kv_heads, (hq // kv_heads) * nq, d)
    qsum = rows[:, :, 0].copy()
    qabs = np.abs(rows[:, :, 0])
    for r in range(1, rows.shape[2]):
        qsum = (qsum + rows[:, :, r]).astype(np.float32)
        qabs = (qabs + np.abs(rows[:, :, r])).astype(np.float32)
    return qsum, qabs


def page_scores(query: np.ndarray, kmin: np.ndarray, kmax: np.ndarray, max_done: int) -> np.ndarray:
    """``[B, Hkv, max_done]`` fp32 upper-bound scores of the pages (quest.py:93-98)."""
    qsum, qabs = query_sums(query, kmin.shape[1])
    lo = np.asarray(kmin[:, :, :max_done], dtype=np.float32)
    hi = np.asarray(kmax[:, :, :max_done], dtype=np.float32)
    mid = ((lo + hi).astype(np.float32) * np.float32(0.5)).astype(np.float32)
    half = ((hi - lo).astype(np.float32) * np.float32(0.5)).astype(np.float32)
    first = tree_dot(qsum[:, :, None, :], mid)
    second = tree_dot(qabs[:, :, None, :], half)
    return (first + second).astype(np.float32)


def select_pages(query: np.ndarray, kmin: np.ndarray, kmax: np.ndarray, done: np.ndarray, max_done: int,
                 pages: int, first_page: bool = False) -> np.ndarray:
    """``int32`` ``[B, Hkv, pages]``: the selected pages of every row and KV head in increasing order, then ``-1``
    (quest.py:73-108, ties to the lower index). ``first_page`` gives page 0 of a row the score +inf (a build option,
    not the reference's rule)."""
    batch, kv_heads = kmin.shape[:2]
    out = np.full((batch, kv_heads, max(pages, 0)), -1, dtype=np.int32)
    if max_done <= 0 or pages <= 0:
        return out
    score = page_scores(query, kmin, kmax, max_done)
    done = np.asarray(done).astype(np.int64)
    count = min(pages, max_done)
    for b in range(batch):
        for h in range(kv_heads):
            s = score[b, h].astype(np.float64)
            s[done[b]:] = -np.inf
            if first_page and done[b] > 0:
                s[0] = np.inf
            order = np.argsort(-s, kind="stable")[:count]
            chosen = np.sort(order[order < done[b]])
            out[b, h, : chosen.size] = chosen
    return out


def keep_slots(index: np.ndarray, done: np.ndarray, page: int, slots: int) -> np.ndarray:
    """Boolean ``[B, Hkv, slots]``: the selected pages' slots and every slot from ``done[b] * page`` on
    (quest.py:145-154)."""
    batch, kv_heads, _ = index.shape
    keep = np.zeros((batch, kv_heads, slots), dtype=bool)
    for b in range(batch):
        for h in range(kv_heads):
            for p in index[b, h]:
                if p >= 0:
                    keep[b, h, p * page: (p + 1) * page] = True
        keep[b, :, int(done[b]) * page:] = True
    return keep


def quest_reference(query: np.ndarray, key: np.ndarray, value: np.ndarray, mask: np.ndarray | None, scale: float,
                    index: np.ndarray, done: np.ndarray, page: int, softcap: float | None = None,
                    sinks: np.ndarray | None = None) -> np.ndarray:
    """Attention over the selected pages and the dense tail (quest.py:207-219 through ``restrict_mask``,
    quest.py:160-189): ``[B, Q, Hq, Dv]`` float32."""
    batch, q_heads, queries, _ = query.shape
    slots = key.shape[2]
    keep = keep_slots(index, done, page, slots)
    keep = np.repeat(keep, q_heads // key.shape[1], axis=1)[:, :, None, :]
    full = np.ones((batch, q_heads, queries, slots), dtype=bool) if mask is None else \
        np.broadcast_to(mask[..., :slots], (batch, q_heads, queries, slots))
    return reference_attention(query, key, value, full & keep, scale, softcap=softcap, sinks=sinks)
