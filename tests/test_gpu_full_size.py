"""Parity at the benchmark shapes: every configuration at its full size, checked on sampled batch rows.

* fp8 e4m3 paged decode at the Llama-3-8B decode shape (B=32, Hq=32, Hkv=8, D=128, 16-token pages in a shuffled
  pool, per-head scales): every row at L=4096, and lengths drawn uniformly from [1024, 8192] (seed 100, the bench's
  ragged draw);
* KIVI int2 and int4 decode: B=16, Hq=32, Hkv=8, D=128, L=8192, 4 of 128 key channels scaled by 10;
* Quest: B=8, Hq=32, Hkv=8, D=128, L=32768 bf16, 32 planted pages per (row, KV head), 63 pages + the tail: the
  selection of every row, the attention of sampled rows;
* KIVI int4 speculative verification: B=64, Q=8, Hq=64, Hkv=8, D=128, L ~ U[1024, 4096].

The caches are filled by the GPU kernels (append, quantize) from bf16 inputs drawn on the CPU. For the sampled rows
the stored codes (and KIVI scales and zero points) are compared bit for bit with the oracle's, and the outputs with
the fp32 definition (attention/decode.py:66-103) over the oracle's decoded cache at atol 2e-3 / rtol 1e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import paged as opaged
from oracle import quest as oquest
from oracle.attention import reference_attention
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
B, HQ, HKV, D, PAGE = 32, 32, 8, 128, 16


def _rows(batch: int) -> list[int]:
    return sorted({0, batch // 3, batch // 2 + 1, batch - 1})


def _fp8_rows_of_cache(cache, table: np.ndarray, b: int, n: int) -> tuple[np.ndarray, np.ndarray]:
    """The stored bytes of row b's n tokens, [Hkv, n, D] each (keys [P, H, D/16, 16, 16], values [P, H, D, 16])."""
    pages = torch.from_numpy(table[b, : -(-n // PAGE)].astype(np.int64)).cuda()
    kc = cache.keys[pages].view(torch.uint8).cpu().numpy()
    vc = cache.values[pages].view(torch.uint8).cpu().numpy()
    k = kc.transpose(1, 0, 3, 2, 4).reshape(HKV, -1, D)[:, :n]
    v = vc.transpose(1, 0, 3, 2).reshape(HKV, -1, D)[:, :n]
    return k, v


@pytest.mark.parametrize("lens_kind", ["fixed_4096", "ragged_1024_8192"])
def test_fp8_decode_at_the_llama3_8b_shape(lens_kind) -> None:
    from economize_amd.paged import PagedKVCache, head_scales, paged_append, paged_decode_attention

    lens = [4096] * B if lens_kind == "fixed_4096" else \
        np.random.default_rng(100).integers(1024, 8193, B).tolist()
    gen = torch.Generator().manual_seed(7)
    smax = max(lens)
    q = torch.randn(B, 1, HQ, D, generator=gen).to(torch.bfloat16)
    k = torch.randn(B, HKV, smax, D, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, HKV, smax, D, generator=gen).to(torch.bfloat16)
    held = (torch.arange(smax)[None, :] < torch.tensor(lens)[:, None])[:, None, :, None]
    k = torch.where(held, k, 0)
    v = torch.where(held, v, 0)
    table, pages = opaged.shuffled_block_table(lens, PAGE, seed=8)
    kd_gpu, vd_gpu = k.cuda(), v.cuda()
    ks, vs = head_scales(kd_gpu), head_scales(vd_gpu)
    cache = PagedKVCache.empty(pages, HKV, D, torch.float8_e4m3fn, "cuda", ks, vs)
    table_gpu = torch.from_numpy(table).cuda()
    for b, n in enumerate(lens):
        t = torch.arange(n, device="cuda")
        slots = (table_gpu[b, t // PAGE] * PAGE + t % PAGE).to(torch.int32)
        paged_append(cache, kd_gpu[b, :, :n].transpose(0, 1), vd_gpu[b, :, :n].transpose(0, 1), slots)
    del kd_gpu, vd_gpu
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = paged_decode_attention(q.cuda(), cache, table_gpu, seq, smax).float().cpu().numpy()

    want_ks = ofp8.head_scales(k.float().numpy(), "e4m3")
    want_vs = ofp8.head_scales(v.float().numpy(), "e4m3")
    assert np.array_equal(ks.cpu().numpy(), want_ks) and np.array_equal(vs.cpu().numpy(), want_vs)
    for b in _rows(B):
        n = lens[b]
        kc, vc = _fp8_rows_of_cache(cache, table, b, n)
        want_kc = ofp8.fp8_encode(k[b, :, :n].float().numpy(), "e4m3", want_ks.reshape(-1, 1, 1))
        want_vc = ofp8.fp8_encode(v[b, :, :n].float().numpy(), "e4m3", want_vs.reshape(-1, 1, 1))
        assert np.array_equal(kc, want_kc) and np.array_equal(vc, want_vc), b
        kf = ofp8.fp8_decode(want_kc[None], "e4m3", want_ks.reshape(1, -1, 1, 1), "f32")
        vf = ofp8.fp8_decode(want_vc[None], "e4m3", want_vs.reshape(1, -1, 1, 1), "f32")
        qb = q[b:b + 1].float().numpy().transpose(0, 2, 1, 3)
        want = reference_attention(qb, kf, vf, None, 1 / np.sqrt(D))
        np.testing.assert_allclose(out[b:b + 1], want, atol=ATOL, rtol=RTOL)


def _kivi_full(batch, queries, q_heads, lens, bits, seed):
    from test_gpu_kivi import device_cache, make_case, oracle_blocks, oracle_output

    from economize_amd.kivi import kivi_decode_attention

    c = make_case(batch, queries, q_heads, HKV, D, lens, bits, seed=seed)
    cache, table = device_cache(c)
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, max(lens)).float().cpu().numpy()
    rows = _rows(batch)
    blocks = cache.blocks.cpu().numpy()
    want_blocks = oracle_blocks(c, D, rows)
    for b in rows:
        pages = c.table[b, : -(-lens[b] // 32)]
        assert np.array_equal(blocks[pages], want_blocks[pages]), b
    want = oracle_output(c, rows=rows)
    np.testing.assert_allclose(got[rows], want[rows], atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("bits", [2, 4])
def test_kivi_decode_at_b16_l8192(bits) -> None:
    _kivi_full(16, 1, HQ, [8192] * 16, bits, seed=60 + bits)


def test_kivi_int4_verification_at_b64_q8() -> None:
    lens = np.random.default_rng(200).integers(1024, 4097, 64).tolist()
    _kivi_full(64, 8, 64, lens, 4, seed=70)


def test_quest_at_b8_l32768_planted() -> None:
    from paged_cases import make_case, to_numpy_f32

    from economize_amd.quest import QuestPages, paged_page_bounds

    batch, length, planted, budget = 8, 32768, 32, 1024
    c = make_case(batch, 1, HQ, HKV, D, [length] * batch, torch.bfloat16, seed=90)
    rng = np.random.default_rng(91)
    k = bf16_bits_to_f32(c.k_codes)
    q = to_numpy_f32(c.q)  # [B, 1, Hq, D]
    for b in range(batch):
        for h in range(HKV):
            for p in rng.choice(length // PAGE - 1, planted, replace=False):
                k[b, h, p * PAGE:(p + 1) * PAGE] = q[b, 0, h * (HQ // HKV)] + 0.1 * rng.standard_normal((PAGE, D))
    c.k_codes = f32_to_bf16_bits(k)
    k = bf16_bits_to_f32(c.k_codes)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    done = np.full(batch, (length - 1) // PAGE, np.int32)
    max_done = int(done.max())
    pages = budget // PAGE - 1
    kmin, kmax = paged_page_bounds(cache, table, 0, max_done, PAGE)
    qp = QuestPages(kmin, kmax, torch.from_numpy(done).cuda(), int(done.min()), max_done, PAGE, pages)
    query = c.q.cuda().transpose(1, 2)  # [B, Hq, 1, D]
    seq = torch.full((batch,), length, dtype=torch.int32, device="cuda")
    got_index = qp.select(query).cpu().numpy()
    got = qp.attend_paged(query, cache, table, seq, length).float().cpu().numpy()

    qn = q.transpose(0, 2, 1, 3)
    lo, hi = oquest.page_bounds(k, 0, max_done, PAGE)
    assert np.array_equal(kmin.cpu().float().numpy(), lo) and np.array_equal(kmax.cpu().float().numpy(), hi)
    index = oquest.select_pages(qn, lo, hi, done, max_done, pages)
    assert np.array_equal(got_index, index)
    vd = bf16_bits_to_f32(c.v_codes)
    for b in _rows(batch):
        want = oquest.quest_reference(qn[b:b + 1], k[b:b + 1], vd[b:b + 1], None, 1 / np.sqrt(D), index[b:b + 1],
                                      done[b:b + 1], PAGE)
        np.testing.assert_allclose(got[b:b + 1], want, atol=ATOL, rtol=RTOL)
