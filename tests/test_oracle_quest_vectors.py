"""The Quest oracle against the reference's own selections (``tests/golden/quest_select_vectors.npz``, written by the
reference's ``page_bounds`` / ``select_pages`` on the CPU, attention/quest.py:54-65, 73-108).

Every case's indices equal the reference's except two, which the definition leaves open: in the exact-tie case the
reference's ``torch.topk`` keeps higher-index members of tied groups (the selected scores are the reference's and
ties go to the lower page index here); in the near-tie case pages whose scores differ by about one fp32 unit are
ordered by the rounding of torch's CPU einsum, whose summation order differs from the fixed order this path uses
(the score bits differ there: parity unpinned at fp32-unit near ties), and every page the two selections disagree on
lies within the fp32 error bound of the k-th score. A selection with ``qsum`` and ``qabs`` swapped or the half-width
term dropped fails the random cases.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quest as oquest
from quest_vectors import check_selection, load

VECTORS = load()


@pytest.mark.parametrize("v", VECTORS, ids=[v.name for v in VECTORS])
def test_oracle_selection_equals_the_reference(v) -> None:
    got = oquest.select_pages(v.query, v.kmin, v.kmax, v.done, v.max_done, v.pages)
    check_selection(v, got)
    if v.name not in ("exact_ties", "near_ties"):
        assert np.array_equal(got, v.index)


def test_the_vectors_hold_ties_and_near_ties() -> None:
    """The tie cases test what they claim: the exact-tie case has tied scores at its k-th place and the reference
    broke at least one of them away from the lower index; the near-tie case has pages within one fp32 unit of its
    k-th score."""
    by = {v.name: v for v in VECTORS}
    ties = by["exact_ties"]
    got = oquest.select_pages(ties.query, ties.kmin, ties.kmax, ties.done, ties.max_done, ties.pages)
    assert not np.array_equal(got, ties.index)
    near = by["near_ties"]
    s = oquest.page_scores(near.query, near.kmin, near.kmax, near.max_done)
    for b in range(s.shape[0]):
        for h in range(s.shape[1]):
            row = np.sort(s[b, h])[::-1]
            kth = row[near.pages - 1]
            close = np.abs(row - kth) <= np.spacing(np.float32(abs(kth)))
            assert close.sum() >= 2


@pytest.mark.parametrize("v", [v for v in VECTORS if v.name == "random_d128"], ids=["random_d128"])
def test_planted_mistakes_fail_the_vectors(v) -> None:
    """Selections with the half-width term dropped, or with ``qsum`` and ``qabs`` swapped, miss the reference's."""
    qsum, qabs = oquest.query_sums(v.query, v.kmin.shape[1])
    mid = (v.kmin[:, :, :v.max_done] + v.kmax[:, :, :v.max_done]) * np.float32(0.5)
    half = (v.kmax[:, :, :v.max_done] - v.kmin[:, :, :v.max_done]) * np.float32(0.5)
    for score in (oquest.tree_dot(qsum[:, :, None], mid), oquest.tree_dot(qabs[:, :, None], mid)
                  + oquest.tree_dot(qsum[:, :, None], half)):
        score = score.astype(np.float64)
        wrong = np.full_like(v.index, -1)
        for b in range(score.shape[0]):
            for h in range(score.shape[1]):
                s = score[b, h].copy()
                s[v.done[b]:] = -np.inf
                k = min(v.pages, v.max_done)
                order = np.argsort(-s, kind="stable")[:k]
                chosen = np.sort(order[order < v.done[b]])
                wrong[b, h, :chosen.size] = chosen
        assert not np.array_equal(wrong, v.index)
