"""Loader of the Quest selection vectors the reference's own ``select_pages`` wrote on the CPU
(``tests/golden/quest_select_vectors.npz``, made by ``tests/golden/make_quest_vectors.py``), and the comparison
both the oracle and the kernels are held to."""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

from oracle import quest as oquest
from oracle.numerics import bf16_bits_to_f32

VECTORS = Path(__file__).resolve().parent / "golden" / "quest_select_vectors.npz"


@dataclass
class QuestVector:
    name: str
    query_bits: np.ndarray  # uint16 bf16 [B, Hq, Q, D]
    kmin_bits: np.ndarray  # uint16 bf16 [B, Hkv, P, D]
    kmax_bits: np.ndarray
    done: np.ndarray  # int32 [B]
    max_done: int
    pages: int
    index: np.ndarray  # int32 [B, Hkv, pages]: the reference's selection

    @property
    def query(self) -> np.ndarray:
        return bf16_bits_to_f32(self.query_bits)

    @property
    def kmin(self) -> np.ndarray:
        return bf16_bits_to_f32(self.kmin_bits)

    @property
    def kmax(self) -> np.ndarray:
        return bf16_bits_to_f32(self.kmax_bits)


def load() -> list[QuestVector]:
    z = np.load(VECTORS)
    names = sorted({k.rsplit("_", 1)[0] for k in z.files if k.endswith("_meta")})
    out = []
    for n in names:
        max_done, pages = (int(x) for x in z[f"{n}_meta"])
        out.append(QuestVector(n, z[f"{n}_query"], z[f"{n}_kmin"], z[f"{n}_kmax"], z[f"{n}_done"], max_done, pages,
                               z[f"{n}_index"]))
    return out


def near_tie_slack(v: QuestVector) -> tuple[np.ndarray, np.ndarray]:
    """``(exact, bound)`` ``[B, Hkv, max_done]``: the pages' scores in float64 from the fp32 group sums and bounds, and
    the forward error bound of any fp32 summation order of the score's ``2 D`` products (``gamma_{2D+1}`` times the
    sum of their magnitudes)."""
    qsum, qabs = oquest.query_sums(v.query, v.kmin.shape[1])
    lo = v.kmin[:, :, :v.max_done].astype(np.float64)
    hi = v.kmax[:, :, :v.max_done].astype(np.float64)
    mid, half = (lo + hi) * 0.5, (hi - lo) * 0.5
    a, b = qsum[:, :, None, :].astype(np.float64), qabs[:, :, None, :].astype(np.float64)
    exact = (a * mid + b * half).sum(-1)
    n = 2 * v.kmin.shape[3] + 1
    u = 2.0 ** -24
    bound = n * u / (1 - n * u) * (np.abs(a * mid) + np.abs(b * half)).sum(-1)
    return exact, bound


def check_selection(v: QuestVector, got: np.ndarray) -> None:
    """``got`` equals the reference's selection, except where the choice is not fixed by the definition:

    * among pages of exactly equal score the reference's ``torch.topk`` keeps an unspecified member of a tied group
      and this path the lowest page index: there the selected scores must be the same multiset as the reference's,
      and every page passed over for a tied page must have the higher index;
    * at near ties (scores within the fp32 error bound of the k-th score) the reference's bits follow its backend's
      einsum order: every page that one selection holds and the other does not must lie within the error bound of
      the k-th exact score."""
    assert got.shape == v.index.shape
    if np.array_equal(got, v.index):
        return
    if v.name == "near_ties":
        exact, bound = near_tie_slack(v)
        for b in range(got.shape[0]):
            for h in range(got.shape[1]):
                g, w = set(got[b, h][got[b, h] >= 0].tolist()), set(v.index[b, h][v.index[b, h] >= 0].tolist())
                assert len(g) == len(w), (v.name, b, h)
                if g == w:
                    continue
                kth = np.sort(exact[b, h, :v.done[b]])[::-1][len(w) - 1]
                for p in g ^ w:
                    assert abs(exact[b, h, p] - kth) <= 2 * bound[b, h, p], (v.name, b, h, p, "not a near tie")
        return
    score = oquest.page_scores(v.query, v.kmin, v.kmax, v.max_done)
    for b in range(got.shape[0]):
        for h in range(got.shape[1]):
            g, w = got[b, h], v.index[b, h]
            if np.array_equal(g, w):
                continue
            assert (g >= 0).sum() == (w >= 0).sum(), (v.name, b, h, g, w)
            gs = np.sort(score[b, h, g[g >= 0]])
            ws = np.sort(score[b, h, w[w >= 0]])
            assert np.array_equal(gs, ws), (v.name, b, h, "selected scores differ", g, w)
            kept = set(g[g >= 0].tolist())
            for p in set(w[w >= 0].tolist()) - kept:  # the reference kept p, this path a tied page instead
                tied = [x for x in kept - set(w.tolist()) if score[b, h, x] == score[b, h, p]]
                assert tied and min(tied) < p, (v.name, b, h, p, "a tie not broken toward the lower page")
