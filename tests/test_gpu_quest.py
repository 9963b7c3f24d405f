"""Parity of the Quest kernels with the oracle on the GPU.

* page bounds: bit-exact against ``page_bounds`` (attention/quest.py:54-65) over the stored keys read back from the
  pages (fp8 decoded exactly), for Quest pages of 16 and 32 tokens;
* selection: the selected page indices equal the oracle's ``select_pages`` (attention/quest.py:73-108, summation order
  and ties fixed as in oracle/quest.py), including rows with no more committed pages than the budget, tied scores and
  several query rows per KV head;
* attention over the selected pages and the dense tail within atol 2e-3 / rtol 1e-2 of ``quest_reference``
  (attention/quest.py:207-219), and the selection of the planted-page workload equals the oracle's.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import quest as oquest
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits
from paged_cases import FMT_NAME, make_case, to_numpy_f32

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _stored_keys(case) -> np.ndarray:
    """The keys as the cache stores them, float32 ``[B, Hkv, S, D]`` (fp8 bytes decoded exactly, no scale)."""
    if case.dtype == torch.bfloat16:
        return bf16_bits_to_f32(case.k_codes)
    return ofp8.fp8_decode(case.k_codes, FMT_NAME[case.dtype], None, "f32")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("page", [16, 32])
def test_page_bounds_match_the_oracle(dtype, page) -> None:
    from economize_amd.quest import paged_page_bounds

    lens = [700, 64, 1025, 130]
    c = make_case(4, 1, 16, 4, 128, lens, dtype, seed=31)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    last = max(lens) // page
    kmin, kmax = paged_page_bounds(cache, table, 0, last, page)
    torch.cuda.synchronize()
    want_lo, want_hi = oquest.page_bounds(_stored_keys(c), 0, last, page)
    got_lo, got_hi = kmin.float().cpu().numpy(), kmax.float().cpu().numpy()
    for b, n in enumerate(lens):
        full = n // page  # pages every token of which the row holds
        assert np.array_equal(got_lo[b, :, :full], want_lo[b, :, :full])
        assert np.array_equal(got_hi[b, :, :full], want_hi[b, :, :full])


def test_page_bounds_update_a_window_in_place() -> None:
    """Bounds of pages [first, last) written into existing tensors, the others untouched (the incremental update of
    techniques/quest/technique.py:229-259)."""
    from economize_amd.quest import paged_page_bounds

    c = make_case(2, 1, 8, 2, 64, [512, 400], torch.float8_e4m3fn, seed=3)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    kmin = torch.full((2, 2, 32, 64), 7.0, dtype=torch.bfloat16, device="cuda")
    kmax = kmin.clone()
    paged_page_bounds(cache, table, 5, 20, 16, out=(kmin, kmax))
    want_lo, want_hi = oquest.page_bounds(_stored_keys(c), 0, 25, 16)
    lo = kmin.float().cpu().numpy()
    assert np.array_equal(lo[:, :, 5:20], want_lo[:, :, 5:20])
    assert (lo[:, :, :5] == 7).all() and (lo[:, :, 20:] == 7).all()
    assert np.array_equal(kmax.float().cpu().numpy()[:, :, 5:20], want_hi[:, :, 5:20])


def _random_bounds(rng, batch, kv_heads, pages, d):
    lo = rng.standard_normal((batch, kv_heads, pages, d)).astype(np.float32)
    hi = lo + np.abs(rng.standard_normal((batch, kv_heads, pages, d))).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(lo)), bf16_bits_to_f32(f32_to_bf16_bits(hi))


def _to_bf16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(f32_to_bf16_bits(x).view(np.int16)).view(torch.bfloat16).cuda()


@pytest.mark.parametrize("shape", [
    # batch, q heads, kv heads, queries, head dim, bound pages, selected pages
    (3, 32, 8, 1, 128, 300, 63),
    (2, 8, 8, 1, 64, 40, 9),
    (2, 16, 4, 2, 128, 2048, 63),
    (2, 8, 2, 1, 256, 77, 100),  # more pages asked than exist
    (2, 8, 2, 1, 128, 4096, 127),  # 16 keys per selecting thread
    (1, 4, 1, 3, 64, 5000, 255),
    (2, 8, 2, 1, 512, 100, 20),  # 64 lanes per page, 16 pages per scoring workgroup
    (1, 4, 1, 1, 64, 20000, 511),  # more committed pages than the selection holds in LDS
])
def test_selection_matches_the_oracle(shape) -> None:
    from economize_amd.quest import select_pages

    batch, hq, hkv, nq, d, npages, pages = shape
    rng = np.random.default_rng(sum(shape))
    lo, hi = _random_bounds(rng, batch, hkv, npages, d)
    q = bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal((batch, hq, nq, d)).astype(np.float32)))
    done = rng.integers(0, npages + 1, batch).astype(np.int32)
    done[0] = npages
    if batch > 1:
        done[1] = min(pages, npages) // 2  # fewer committed pages than the budget: all of them
    max_done = int(done.max())
    got = select_pages(_to_bf16(q), _to_bf16(lo), _to_bf16(hi), torch.from_numpy(done).cuda(), max_done, pages)
    want = oquest.select_pages(q, lo, hi, done, max_done, pages)
    assert np.array_equal(got.cpu().numpy(), want)


def test_tied_scores_go_to_the_lower_page() -> None:
    from economize_amd.quest import select_pages

    rng = np.random.default_rng(4)
    lo, hi = _random_bounds(rng, 1, 1, 64, 128)
    lo[0, 0, 40:] = lo[0, 0, 10]  # pages 10 and 40..63 score the same
    hi[0, 0, 40:] = hi[0, 0, 10]
    q = bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal((1, 4, 1, 128)).astype(np.float32)))
    done = np.array([64], np.int32)
    for pages in (3, 10, 20, 30):
        got = select_pages(_to_bf16(q), _to_bf16(lo), _to_bf16(hi), torch.from_numpy(done).cuda(), 64, pages)
        want = oquest.select_pages(q, lo, hi, done, 64, pages)
        assert np.array_equal(got.cpu().numpy(), want), pages


def test_selection_narrows_crowded_buckets() -> None:
    """Score distributions that crowd the bucket of the threshold: 1500 tied pages above the rest (the threshold is
    their one value), a row whose pages all tie, and a cluster of 500 distinct scores between 10 far outliers and one
    far negative page (at 255 pages the threshold's bucket of the whole range holds 394 keys, which are counted again
    over their own range before they are ranked)."""
    from economize_amd.quest import select_pages

    rng = np.random.default_rng(9)
    lo, hi = _random_bounds(rng, 3, 1, 2000, 128)
    q = bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal((3, 4, 1, 128)).astype(np.float32)))
    lo[0, 0, 300:1800] = lo[0, 0, 5]
    hi[0, 0, 300:1800] = lo[0, 0, 5] + 3.0
    lo[1, 0, :] = lo[1, 0, 0]
    hi[1, 0, :] = hi[1, 0, 0]
    hi[2, 0, 0:10] += 500.0
    hi[2, 0, 100:600] = lo[2, 0, 100:600] + 5.0 + 0.01 * rng.standard_normal((500, 128)).astype(np.float32)
    lo[2, 0, 1999] = hi[2, 0, 1999] = -500.0 * np.sign(q[2].sum(axis=(0, 1)))
    lo, hi = bf16_bits_to_f32(f32_to_bf16_bits(lo)), bf16_bits_to_f32(f32_to_bf16_bits(hi))
    done = np.array([2000, 2000, 2000], np.int32)
    for pages in (63, 255):
        got = select_pages(_to_bf16(q), _to_bf16(lo), _to_bf16(hi), torch.from_numpy(done).cuda(), 2000, pages)
        want = oquest.select_pages(q, lo, hi, done, 2000, pages)
        assert np.array_equal(got.cpu().numpy(), want), pages


def test_no_committed_pages_selects_nothing() -> None:
    from economize_amd.quest import select_pages

    q = torch.zeros(2, 4, 1, 64, dtype=torch.bfloat16, device="cuda")
    bounds = torch.zeros(2, 1, 4, 64, dtype=torch.bfloat16, device="cuda")
    got = select_pages(q, bounds, bounds, torch.zeros(2, dtype=torch.int32, device="cuda"), 0, 5)
    assert (got.cpu().numpy() == -1).all()


@pytest.mark.parametrize("dtype,page", [(torch.bfloat16, 16), (torch.float8_e4m3fn, 16), (torch.bfloat16, 32)])
def test_quest_attention_matches_the_oracle(dtype, page) -> None:
    from economize_amd.quest import QuestPages, paged_page_bounds

    lens = [3000, 900, 2500]
    c = make_case(3, 1, 32, 8, 128, lens, dtype, seed=41 + page)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    done = np.array([(n - 1) // page for n in lens], np.int32)
    max_done = int(done.max())
    pages = 1024 // page - 1
    kmin, kmax = paged_page_bounds(cache, table, 0, max_done, page)
    qp = QuestPages(kmin, kmax, torch.from_numpy(done).cuda(), int(done.min()), max_done, page, pages)
    query = c.q.cuda().transpose(1, 2)  # [B, Hq, 1, D]
    got = qp.attend_paged(query, cache, table, seq, max(lens)).float().cpu().numpy()
    q = to_numpy_f32(c.q).transpose(0, 2, 1, 3)
    lo, hi = oquest.page_bounds(_stored_keys(c), 0, max_done, page)
    index = oquest.select_pages(q, lo, hi, done, max_done, pages)
    assert np.array_equal(qp.select(query).cpu().numpy(), index)
    kd, vd = c.decoded()
    visible = (np.arange(kd.shape[2])[None, :] < np.array(lens)[:, None])[:, None, None, :]
    want = oquest.quest_reference(q, kd, vd, visible, 1 / np.sqrt(128), index, done, page)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


def test_planted_workload_selection_matches_the_oracle() -> None:
    """The Quest decode workload: keys of 32 planted pages per (row, KV head) are the group's first query plus
    0.1 N(0, 1). The selection equals the oracle's. (Quest's score is an upper bound: a planted page's keys are
    close together, so its bound's width term is small, and random pages with wide bounds can outrank it.)"""
    from economize_amd.quest import paged_page_bounds, select_pages

    batch, hq, hkv, d, length, page = 2, 32, 8, 128, 4096, 16
    c = make_case(batch, 1, hq, hkv, d, [length] * batch, torch.bfloat16, seed=9)
    rng = np.random.default_rng(10)
    k = to_numpy_f32(c.k)
    q = to_numpy_f32(c.q)  # [B, 1, Hq, D]
    for b in range(batch):
        for h in range(hkv):
            for p in rng.choice(length // page - 1, 32, replace=False):
                k[b, h, p * page:(p + 1) * page] = q[b, 0, h * (hq // hkv)] + 0.1 * rng.standard_normal((page, d))
    c.k_codes = f32_to_bf16_bits(k)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    done = np.full(batch, (length - 1) // page, np.int32)
    kmin, kmax = paged_page_bounds(cache, table, 0, int(done[0]), page)
    got = select_pages(c.q.cuda().transpose(1, 2), kmin, kmax, torch.from_numpy(done).cuda(), int(done[0]), 63)
    lo, hi = oquest.page_bounds(bf16_bits_to_f32(c.k_codes), 0, int(done[0]), page)
    want = oquest.select_pages(q.transpose(0, 2, 1, 3), lo, hi, done, int(done[0]), 63)
    assert np.array_equal(got.cpu().numpy(), want)


def test_quest_attention_with_a_mask() -> None:
    """A mask hides keys of the selected pages and of the tail alike (the reference's Quest kernel reads the mask,
    attention/_quest_kernels.py:55-87)."""
    from economize_amd.quest import QuestPages, paged_page_bounds

    lens, page = [3000, 900, 2500], 16
    c = make_case(3, 1, 32, 8, 128, lens, torch.float8_e4m3fn, seed=43)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    done = np.array([(n - 1) // page for n in lens], np.int32)
    max_done = int(done.max())
    kmin, kmax = paged_page_bounds(cache, table, 0, max_done, page)
    qp = QuestPages(kmin, kmax, torch.from_numpy(done).cuda(), int(done.min()), max_done, page, 63)
    mask = np.random.default_rng(44).random((3, 1, 1, max(lens))) < 0.7
    query = c.q.cuda().transpose(1, 2)
    got = qp.attend_paged(query, cache, table, seq, max(lens), mask=torch.from_numpy(mask).cuda()).float().cpu().numpy()
    q = to_numpy_f32(c.q).transpose(0, 2, 1, 3)
    lo, hi = oquest.page_bounds(_stored_keys(c), 0, max_done, page)
    index = oquest.select_pages(q, lo, hi, done, max_done, 63)
    kd, vd = c.decoded()
    visible = (np.arange(kd.shape[2])[None, :] < np.array(lens)[:, None])[:, None, None, :] & mask
    want = oquest.quest_reference(q, kd, vd, visible, 1 / np.sqrt(128), index, done, page)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("shape", [(2, 8, 2, 1, 128, 64, 8), (1, 4, 1, 1, 64, 3000, 63)])
def test_forced_first_page_matches_the_oracle(shape) -> None:
    """``first_page`` selects page 0 of every row with a committed page, also where it scores lowest."""
    from economize_amd.quest import select_pages

    batch, hq, hkv, nq, d, npages, pages = shape
    rng = np.random.default_rng(7 + npages)
    lo, hi = _random_bounds(rng, batch, hkv, npages, d)
    q = bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal((batch, hq, nq, d)).astype(np.float32)))
    qsum = q[0, :, 0].reshape(hkv, hq // hkv, d).sum(1)
    lo[0, :, 0] = hi[0, :, 0] = bf16_bits_to_f32(f32_to_bf16_bits(-8.0 * np.sign(qsum).astype(np.float32)))
    done = np.full(batch, npages, np.int32)
    if batch > 1:
        done[1] = 0  # nothing committed: nothing selected
    got = select_pages(_to_bf16(q), _to_bf16(lo), _to_bf16(hi), torch.from_numpy(done).cuda(), npages, pages,
                       first_page=True)
    want = oquest.select_pages(q, lo, hi, done, npages, pages, first_page=True)
    assert np.array_equal(got.cpu().numpy(), want)
    assert (want[0, :, 0] == 0).all()
    plain = oquest.select_pages(q, lo, hi, done, npages, pages)
    assert not (plain[0, :, 0] == 0).any()  # the planted page 0 is selected only when forced


def _vector_ids():
    from quest_vectors import load

    return [v.name for v in load()]


@pytest.mark.parametrize("name", _vector_ids())
def test_selection_matches_the_reference_vectors(name) -> None:
    """The selection kernel on the reference's own CPU selections (``tests/golden/quest_select_vectors.npz``):
    indices equal the oracle's bit for bit, and the reference's, up to the tie order and the fp32-unit near ties the
    definition leaves open (``quest_vectors.check_selection``)."""
    from economize_amd.quest import select_pages
    from quest_vectors import check_selection, load

    v = next(x for x in load() if x.name == name)
    bf16 = lambda bits: torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).cuda()  # noqa: E731
    got = select_pages(bf16(v.query_bits), bf16(v.kmin_bits), bf16(v.kmax_bits), torch.from_numpy(v.done).cuda(),
                       v.max_done, v.pages).cpu().numpy()
    want = oquest.select_pages(v.query, v.kmin, v.kmax, v.done, v.max_done, v.pages)
    assert np.array_equal(got, want)
    check_selection(v, got)
