"""Pins the oracle's Quest page bounds, selection and restricted attention (attention/quest.py:54-219)."""

from __future__ import annotations

import numpy as np

from oracle import quest
from oracle.attention import reference_attention


def test_page_bounds_are_channel_extremes() -> None:
    k = np.random.default_rng(0).standard_normal((2, 3, 64, 8)).astype(np.float32)
    lo, hi = quest.page_bounds(k, 1, 4, 16)
    for p in range(3):
        block = k[:, :, (p + 1) * 16: (p + 2) * 16]
        assert np.array_equal(lo[:, :, p], block.min(2)) and np.array_equal(hi[:, :, p], block.max(2))


def test_tree_dot_is_a_dot_product() -> None:
    rng = np.random.default_rng(1)
    for d in (8, 64, 96, 128):
        a, b = rng.standard_normal((5, d)).astype(np.float32), rng.standard_normal((5, d)).astype(np.float32)
        assert np.allclose(quest.tree_dot(a, b), (a.astype(np.float64) * b).sum(-1), rtol=1e-5, atol=1e-5)
    # the order is the documented one: runs of 8, then a halving tree
    a = np.float32([1e8] + [1.0] * 15)
    b = np.ones(16, np.float32)
    run0 = np.float32(1e8)
    for _ in range(7):
        run0 = np.float32(run0 + np.float32(1.0))
    run1 = np.float32(8.0)
    assert quest.tree_dot(a, b) == np.float32(run0 + run1)


def _official_bound(query: np.ndarray, kmin: np.ndarray, kmax: np.ndarray) -> np.ndarray:
    """``sum_h sum_d max(q_hd * lo_d, q_hd * hi_d)`` over the group's heads in float64 (the per-head form of the
    official Quest bound)."""
    b, hq, nq, d = query.shape
    hkv = kmin.shape[1]
    q = query.astype(np.float64).reshape(b, hkv, (hq // hkv) * nq, 1, d)
    lo, hi = kmin.astype(np.float64)[:, :, None], kmax.astype(np.float64)[:, :, None]
    return np.maximum(q * lo, q * hi).sum(-1).sum(2)


def test_selection_equals_the_official_bound_away_from_ties() -> None:
    rng = np.random.default_rng(2)
    checked = 0
    for seed in range(20):
        q = rng.standard_normal((2, 8, 1, 32)).astype(np.float32)
        k = rng.standard_normal((2, 2, 40 * 16, 32)).astype(np.float32)
        lo, hi = quest.page_bounds(k, 0, 40, 16)
        done = np.array([40, 33])
        pages = 7
        got = quest.select_pages(q, lo, hi, done, 40, pages)
        exact = _official_bound(q, lo, hi)
        for b in range(2):
            for h in range(2):
                s = exact[b, h, : done[b]]
                order = np.argsort(-s, kind="stable")
                gap = s[order[pages - 1]] - s[order[pages]]
                if gap < 1e-3 * (1 + np.abs(s).max()):
                    continue  # a near tie: fp32 rounding decides, not pinned
                checked += 1
                assert got[b, h].tolist() == sorted(order[:pages].tolist())
    assert checked > 60


def test_selection_invariants() -> None:
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 8, 1, 16)).astype(np.float32)
    k = rng.standard_normal((2, 2, 100, 16)).astype(np.float32)
    lo, hi = quest.page_bounds(k, 0, 6, 16)
    sel = quest.select_pages(q, lo, hi, np.array([6, 4]), 6, 2)
    assert sel.shape == (2, 2, 2) and (sel[1] < 4).all() and (sel >= 0).all() and (np.diff(sel, axis=-1) > 0).all()
    few = quest.select_pages(q, lo, hi, np.array([6, 1]), 6, 3)
    assert few[1].tolist() == [[0, -1, -1]] * 2  # a short row reads its committed pages, then nothing
    assert (quest.select_pages(q, lo, hi, np.array([0, 0]), 0, 3) == -1).all()


def test_ties_go_to_the_lower_page() -> None:
    q = np.ones((1, 1, 1, 8), np.float32)
    lo = np.zeros((1, 1, 6, 8), np.float32)
    hi = np.zeros((1, 1, 6, 8), np.float32)
    hi[0, 0, [1, 3, 4]] = 1.0  # three equal scores for two picks
    sel = quest.select_pages(q, lo, hi, np.array([6]), 6, 2)
    assert sel.tolist() == [[[1, 3]]]


def test_keep_and_restricted_attention() -> None:
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 4, 1, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 80, 16)).astype(np.float32)
    v = rng.standard_normal((1, 2, 80, 16)).astype(np.float32)
    lo, hi = quest.page_bounds(k, 0, 4, 16)
    index = quest.select_pages(q, lo, hi, np.array([4]), 4, 2)
    keep = quest.keep_slots(index, np.array([4]), 16, 80)
    for h in range(2):
        want = [p * 16 + i for p in index[0, h] for i in range(16)] + list(range(64, 80))
        assert keep[0, h].nonzero()[0].tolist() == want
    got = quest.quest_reference(q, k, v, None, 0.25, index, np.array([4]), 16)
    mask = np.repeat(keep, 2, axis=1)[:, :, None, :]
    assert np.array_equal(got, reference_attention(q, k, v, mask, 0.25))


def test_forced_first_page_is_page_zero_plus_the_rest_by_score() -> None:
    """With ``first_page`` the selection is page 0 plus the selection of ``pages - 1`` among pages 1.. (the same
    rule over the bounds without page 0, shifted back), including a row whose page 0 scores lowest."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 8, 1, 32)).astype(np.float32)
    k = rng.standard_normal((2, 2, 30 * 16, 32)).astype(np.float32)
    lo, hi = quest.page_bounds(k, 0, 30, 16)
    qsum = q[0, :, 0].reshape(2, 4, 32).sum(1)  # per KV head, over its query heads
    lo[0, :, 0] = hi[0, :, 0] = -100.0 * np.sign(qsum)  # row 0: page 0 scores far below every other page
    done, pages = np.array([30, 12]), 6
    got = quest.select_pages(q, lo, hi, done, 30, pages, first_page=True)
    rest = quest.select_pages(q, lo[:, :, 1:], hi[:, :, 1:], done - 1, 29, pages - 1)
    for b in range(2):
        for h in range(2):
            want = [0] + [p + 1 for p in rest[b, h] if p >= 0]
            assert got[b, h].tolist() == want
    assert 0 not in quest.select_pages(q, lo, hi, done, 30, pages)[0, 0].tolist()
    # a row with no committed page selects nothing, forced or not
    assert (quest.select_pages(q, lo, hi, np.array([0, 0]), 30, pages, first_page=True) == -1).all()
