"""The gathered-decode oracle pinned on the CPU: with the compact entries equal to the kept dense entries it is the
dense attention with the evicted prompt entries masked, the reference's statement of the kernel
(attention/gathered.py:12-14); no compact entry with ``start = 0`` is plain dense attention."""

from __future__ import annotations

import numpy as np

from oracle.attention import reference_attention
from oracle.gathered import gathered_reference


def case(seed: int, queries: int = 1, with_mask: bool = False):
    rng = np.random.default_rng(seed)
    b, hq, hkv, s, d, dv = 2, 6, 3, 40, 16, 8
    q = rng.standard_normal((b, hq, queries, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, s, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, s, dv)).astype(np.float32)
    start = np.array([25, 31])
    keep = rng.random((b, hkv, s)) < 0.5
    cap = 32
    ck = np.zeros((b, hkv, cap, d), np.float32)
    cv = np.zeros((b, hkv, cap, dv), np.float32)
    index = np.zeros((b, hkv, cap), np.int32)
    count = np.zeros((b, hkv), np.int32)
    for bb in range(b):
        for h in range(hkv):
            slots = np.nonzero(keep[bb, h, : start[bb]])[0]
            count[bb, h] = len(slots)
            ck[bb, h, : len(slots)], cv[bb, h, : len(slots)] = k[bb, h, slots], v[bb, h, slots]
            index[bb, h, : len(slots)] = slots
    mask = rng.random((b, 1, queries, s)) < 0.8 if with_mask else None
    return q, k, v, mask, ck, cv, index, count, start, keep


def test_compact_entries_equal_the_masked_dense_attention() -> None:
    for seed, queries, with_mask in ((0, 1, False), (1, 3, True), (2, 2, True)):
        q, k, v, mask, ck, cv, index, count, start, keep = case(seed, queries, with_mask)
        got = gathered_reference(q, k, v, mask, 0.3, ck, cv, index, count, start, softcap=5.0)
        evicted = np.ones((2, 6, queries, 40), bool)
        for b in range(2):
            for h in range(3):
                hidden = ~keep[b, h, : start[b]]
                evicted[b, 2 * h: 2 * h + 2, :, : start[b]] &= ~hidden
        full = evicted if mask is None else evicted & np.broadcast_to(mask, evicted.shape)
        want = reference_attention(q, k, v, full, 0.3, softcap=5.0)
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_no_compact_entry_is_dense_attention() -> None:
    q, k, v, mask, ck, cv, index, count, start, _ = case(3, 2, True)
    zeros = np.zeros_like(count)
    got = gathered_reference(q, k, v, mask, 0.25, ck, cv, index, zeros, np.zeros(2, np.int64))
    np.testing.assert_allclose(got, reference_attention(q, k, v, mask, 0.25), rtol=1e-5, atol=1e-6)
