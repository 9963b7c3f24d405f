"""Pins the oracle's paged layout: scatter/gather identity and the element addresses."""

from __future__ import annotations

import numpy as np

from oracle import paged


def test_scatter_gather_identity_and_addresses() -> None:
    rng = np.random.default_rng(0)
    lens = [37, 16, 70]
    table, total = paged.shuffled_block_table(lens, 16, seed=1)
    assert len(set(table[table >= 0].tolist())) == sum(-(-n // 16) for n in lens)
    for element in (1, 2):
        k = rng.integers(1, 200, (3, 2, 70, 32)).astype(np.uint8 if element == 1 else np.uint16)
        v = rng.integers(1, 200, (3, 2, 70, 32)).astype(k.dtype)
        kc, vc = paged.scatter_kv(k, v, lens, table, total, 16, element)
        gk, gv = paged.gather_kv(kc, vc, table, lens, 16)
        for b, n in enumerate(lens):
            assert np.array_equal(gk[b, :, :n], k[b, :, :n]) and np.array_equal(gv[b, :, :n], v[b, :, :n])
        assert (kc != 0).sum() == sum(lens) * 2 * 32 and (vc != 0).sum() == sum(lens) * 2 * 32
        x = 16 // element
        flat_k, flat_v = kc.reshape(-1), vc.reshape(-1)
        for b, h, t, d in [(0, 1, 36, 31), (2, 0, 69, 7), (1, 1, 0, 0)]:
            page, pos = table[b, t // 16], t % 16
            k_off = (((page * 2 + h) * (32 // x) + d // x) * 16 + pos) * x + d % x
            v_off = ((page * 2 + h) * 32 + d) * 16 + pos
            assert flat_k[k_off] == k[b, h, t, d] and flat_v[v_off] == v[b, h, t, d]
    slots = paged.slot_mapping(table, 2, 30, 5, 16)
    assert slots.tolist() == [table[2, t // 16] * 16 + t % 16 for t in range(30, 35)]
