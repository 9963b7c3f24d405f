"""Quest over dense K/V buffers on the GPU (the reference's own cache layout, attention/quest.py:54-344):

* ``page_bounds`` (``eco_quest_dense_bounds``) bit-exact against the oracle's page bounds for bf16 / fp16 / fp32 /
  fp8 keys and pages of 16 / 32 / 64 slots, in the dtype ``bounds_dtype`` names, a window written in place;
* ``select_pages`` with fp16 / fp32 queries and bounds: the oracle's indices (the same fixed fp32 order);
* ``quest_decode_attention`` (``eco_quest_decode``) within atol 2e-3 / rtol 1e-2 of the oracle's
  ``quest_reference`` (the fp32 definition over the selected pages and the tail): query dtypes bf16 / fp16 / fp32,
  fp8 K/V views, head dims 16 to 256 and ``Dv != D``, pages of 16 / 32 / 64 slots, rows with fewer committed pages
  than the budget (``-1`` entries), boolean masks, soft cap, sinks, several queries; with the selected pages given,
  every unselected committed slot holds NaN, so reading one would show;
* ``QuestPages.keep`` / ``restrict_mask`` equal the oracle's kept slots, for boolean, float and absent masks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import quest as oquest

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
FP8 = {torch.float8_e4m3fn: "e4m3", torch.float8_e5m2: "e5m2"}


def _keys(shape, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=gen) * 3
    if dtype in FP8:
        codes = ofp8.fp8_encode(x.numpy(), FP8[dtype], None)
        return torch.from_numpy(codes).view(dtype), ofp8.fp8_decode(codes, FP8[dtype], None, "f32")
    t = x.to(dtype)
    return t, t.float().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float8_e4m3fn,
                                   torch.float8_e5m2])
@pytest.mark.parametrize("page", [16, 32, 64])
def test_dense_page_bounds_are_exact(dtype, page) -> None:
    from economize_amd.quest import bounds_dtype, page_bounds

    keys, kf = _keys((2, 3, 8 * page + 5, 48), dtype, seed=page)
    kmin, kmax = page_bounds(keys.cuda(), 1, 8, page)
    assert kmin.dtype == bounds_dtype(dtype) == (torch.bfloat16 if dtype in FP8 else dtype)
    lo, hi = oquest.page_bounds(kf, 1, 8, page)
    assert np.array_equal(kmin.float().cpu().numpy(), lo) and np.array_equal(kmax.float().cpu().numpy(), hi)
    # a window written in place; the pages outside it keep their values
    lo_all, hi_all = page_bounds(keys.cuda(), 0, 8, page)
    out = (torch.full_like(lo_all, 7.0), torch.full_like(hi_all, 7.0))
    page_bounds(keys.cuda()[:, :, :, :], 3, 6, page, out=out)
    assert torch.equal(out[0][:, :, 3:6], lo_all[:, :, 3:6]) and torch.equal(out[1][:, :, 3:6], hi_all[:, :, 3:6])
    assert bool((out[0][:, :, :3] == 7).all()) and bool((out[1][:, :, 6:] == 7).all())


def test_dense_page_bounds_read_strided_buffers() -> None:
    """The first ``length`` slots of a larger cache buffer (the view a cache layer hands over)."""
    from economize_amd.quest import page_bounds

    keys, kf = _keys((2, 2, 200, 64), torch.float16, seed=3)
    kmin, kmax = page_bounds(keys.cuda()[:, :, :130], 0, 8, 16)
    lo, hi = oquest.page_bounds(kf[:, :, :130], 0, 8, 16)
    assert np.array_equal(kmin.float().cpu().numpy(), lo) and np.array_equal(kmax.float().cpu().numpy(), hi)


@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("kdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_selection_takes_every_query_and_bounds_dtype(qdtype, kdtype) -> None:
    from economize_amd.quest import page_bounds, select_pages

    gen = torch.Generator().manual_seed(11)
    keys, kf = _keys((3, 2, 60 * 16, 64), kdtype, seed=12)
    q = torch.randn(3, 8, 1, 64, generator=gen).to(qdtype)
    done = np.array([60, 33, 9], np.int32)
    kmin, kmax = page_bounds(keys.cuda(), 0, 60, 16)
    got = select_pages(q.cuda(), kmin, kmax, torch.from_numpy(done).cuda(), 60, 12)
    lo, hi = oquest.page_bounds(kf, 0, 60, 16)
    want = oquest.select_pages(q.float().numpy(), lo, hi, done, 60, 12)
    assert np.array_equal(got.cpu().numpy(), want)


CASES = [
    # batch, Hq, Hkv, Q, slots, D, Dv, query dtype, K/V dtype, page, pages, done per row, mask, softcap, sinks
    (3, 8, 2, 1, 1000, 128, 128, torch.bfloat16, torch.bfloat16, 16, 8, [62, 40, 5], None, None, False),
    (2, 4, 2, 1, 40, 16, 16, torch.float32, torch.float32, 16, 1, [2, 2], None, None, False),  # the golden model
    (2, 16, 4, 1, 700, 64, 64, torch.float16, torch.float16, 32, 6, [21, 13], "holes", None, True),
    (2, 8, 2, 1, 2000, 256, 256, torch.bfloat16, torch.bfloat16, 64, 5, [31, 20], None, 30.0, False),
    (2, 12, 4, 1, 900, 128, 128, torch.bfloat16, torch.float8_e4m3fn, 16, 10, [56, 56], "per_head", None, False),
    (2, 8, 8, 1, 333, 96, 64, torch.float32, torch.float32, 16, 4, [20, 7], None, None, True),
    (2, 8, 2, 3, 640, 64, 64, torch.bfloat16, torch.bfloat16, 16, 6, [39, 30], "causal", None, False),
    (1, 32, 8, 1, 4096, 128, 128, torch.float16, torch.float16, 16, 63, [256], None, None, False),
    (2, 4, 1, 1, 129, 48, 48, torch.float32, torch.float8_e5m2, 32, 1, [4, 3], None, None, False),
    (2, 8, 2, 1, 800, 512, 512, torch.bfloat16, torch.bfloat16, 16, 9, [48, 30], "holes", None, True),  # wide heads
    (2, 8, 4, 2, 300, 320, 320, torch.float16, torch.float16, 32, 3, [9, 7], None, None, False),
]


def _case(c, seed):
    batch, hq, hkv, queries, slots, d, dv, qdtype, kvdtype, page, pages, dones, mask_kind, softcap, sinks = c
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    q = torch.randn(batch, queries, hq, d, generator=gen).to(qdtype).transpose(1, 2)  # HF layout
    k, kf = _keys((batch, hkv, slots, d), kvdtype, seed + 1)
    v, vf = _keys((batch, hkv, slots, dv), kvdtype, seed + 2)
    mask = None
    if mask_kind == "holes":
        mask = rng.random((batch, 1, 1, slots)) < 0.8
    elif mask_kind == "per_head":
        mask = rng.random((batch, hq, queries, slots)) < 0.7
    elif mask_kind == "causal":
        mask = np.zeros((batch, 1, queries, slots), bool)
        for qi in range(queries):
            mask[:, :, qi, : slots - queries + qi + 1] = True
    sink = torch.randn(hq, generator=gen) if sinks else None
    return q, k, kf, v, vf, np.array(dones, np.int32), mask, sink


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}h{c[1]}k{c[2]}q{c[3]}s{c[4]}d{c[5]}v{c[6]}-{str(c[7])[6:]}-"
                                             f"{str(c[8])[6:]}-p{c[9]}x{c[10]}-{c[12]}" for c in CASES])
def test_quest_decode_attention_matches_the_oracle(case) -> None:
    from economize_amd.quest import QuestPages, page_bounds, quest_decode_attention

    q, k, kf, v, vf, done, mask, sink = _case(case, seed=len(str(case)))
    page, pages = case[9], case[10]
    softcap = case[13]
    max_done = int(done.max())
    scale = q.shape[-1] ** -0.5
    kmin, kmax = page_bounds(k.cuda(), 0, max_done, page)
    qp = QuestPages(kmin, kmax, torch.from_numpy(done).cuda(), int(done.min()), max_done, page, pages,
                    max_queries=q.shape[2])
    m = None if mask is None else torch.from_numpy(mask).cuda()
    sinks = None if sink is None else sink.cuda()
    got = quest_decode_attention(q.cuda(), k.cuda(), v.cuda(), m, scale, qp, softcap=softcap, sinks=sinks)
    lo, hi = oquest.page_bounds(kf, 0, max_done, page)
    index = oquest.select_pages(q.float().numpy(), lo, hi, done, max_done, pages)
    assert np.array_equal(qp.select(q.cuda()).cpu().numpy(), index)
    want = oquest.quest_reference(q.float().numpy(), kf, vf, mask, scale, index, done, page, softcap=softcap,
                                  sinks=None if sink is None else sink.numpy())
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    # the same pages handed over, every unselected committed slot poisoned
    if k.dtype not in FP8:
        kp, vp = k.clone(), v.clone()
        keep = oquest.keep_slots(index, done, page, k.shape[2])
        for b in range(k.shape[0]):
            for h in range(k.shape[1]):
                hidden = torch.from_numpy(~keep[b, h])
                kp[b, h, hidden] = float("nan")
                vp[b, h, hidden] = float("nan")
        again = quest_decode_attention(q.cuda(), kp.cuda(), vp.cuda(), m, scale, qp, softcap=softcap, sinks=sinks,
                                       index=torch.from_numpy(index).cuda())
        np.testing.assert_allclose(again.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("kind", ["none", "bool", "float", "causal"])
def test_keep_and_restrict_mask_hide_the_unselected_pages(kind) -> None:
    from economize_amd.quest import QuestPages, page_bounds

    gen = torch.Generator().manual_seed(4)
    batch, hq, hkv, slots, d, page, pages = 2, 8, 2, 300, 64, 16, 4
    q = torch.randn(batch, hq, 1, d, generator=gen).to(torch.bfloat16).cuda()
    k = torch.randn(batch, hkv, slots, d, generator=gen).to(torch.bfloat16).cuda()
    done = np.array([18, 3], np.int32)
    kmin, kmax = page_bounds(k, 0, 18, page)
    used = []
    qp = QuestPages(kmin, kmax, torch.from_numpy(done).cuda(), 3, 18, page, pages, on_use=used.append, layer=7)
    index = qp.select(q).cpu().numpy()
    want = oquest.keep_slots(index, done, page, slots)
    assert np.array_equal(qp.keep(q, slots).cpu().numpy(), want)
    full = np.repeat(want, hq // hkv, axis=1)[:, :, None, :]
    if kind == "none":
        got = qp.restrict_mask(q, k, None)
        assert got.dtype == torch.bool and np.array_equal(got.cpu().numpy(), np.broadcast_to(full, got.shape))
    elif kind == "causal":
        got = qp.restrict_mask(q, k, None, is_causal=True)  # one query: the causal mask's first row, top-left
        tril = np.zeros((1, slots), bool)
        tril[0, 0] = True
        assert np.array_equal(got.cpu().numpy(), np.broadcast_to(full & tril, got.shape))
    elif kind == "bool":
        base = torch.rand(batch, 1, 1, slots + 5, generator=gen) < 0.8
        got = qp.restrict_mask(q, k, base.cuda())
        assert np.array_equal(got.cpu().numpy(), np.broadcast_to(full & base[..., :slots].numpy(), got.shape))
    else:
        base = torch.randn(batch, 1, 1, slots, generator=gen).to(torch.bfloat16)
        got = qp.restrict_mask(q, k, base.cuda()).cpu()
        hidden = ~torch.from_numpy(np.broadcast_to(full, got.shape).copy())
        want_f = base.expand(batch, hq, 1, slots).masked_fill(hidden, torch.finfo(torch.bfloat16).min)
        assert torch.equal(got, want_f)
    assert used == [7]
    # a longer query than max_queries sees every key: the mask comes back untouched, and nothing is read
    long_q = torch.randn(batch, hq, 2, d, generator=gen).to(torch.bfloat16).cuda()
    assert qp.restrict_mask(long_q, k, None) is None and used == [7]
